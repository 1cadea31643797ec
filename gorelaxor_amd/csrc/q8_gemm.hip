// q8_gemm.hip - the Q8_0 int8 product for many activation rows (encoder and
// prefill batches, the cross-attention key/value precompute) on the matrix
// cores.
//
// Same arithmetic as q8_gemv.hip, per output (the VNNI kernel's order,
// internal/kern/vnni_amd64.s:58-69 of github.com/xattribution/gorelaxor):
//     c = bias (or 0);  for b in 0..nb-1:  c = fma(f32(s_b) * dw_b, da_b, c)
// Here s_b, the int32 dot of one 32-value block, comes from one
// v_mfma_i32_16x16x32_i8 per 16x16 output tile: its K of 32 is exactly one
// Q8_0 block, so every block's sum stays separate (the K = 64 form would add
// two blocks together before their scales apply).  The lane then folds its
// four int32 results into its four running outputs in block order, so the
// result is bit-identical to the GEMV and to the reference.
//
// A wave computes 16 activation rows x 64 weight rows (one weight tile, four
// MFMAs sharing the A fragment); a workgroup of four waves covers 64 x 64.
// Per block a lane loads 8 bytes of A, 4 x 8 bytes of B (the weight tile
// layout keeps each row's 32 bytes in two 16-byte halves), four weight scales
// and four activation scales.  The per-output fold (convert, multiply, fma:
// 3 VALU ops per output per block) is the bound, not the MFMA: exact
// per-block scaling costs that much vector work per 32 multiply-adds.
#include <cstdint>
#include <cstdlib>
#include <type_traits>

#include "grx_internal.h"
#include "grx_ln.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

// What the epilogue does with each finished output c (GemmOut::epi):
//   STORE      y = c
//   ADD        y = y + c                      (kern.Add of the product)
//   AXPY_HALF  y = fma(0.5, c, y)             (AddScaled(y, c, 0.5), whole groups of 8)
//   SCALE      y = c * scale
//   SILU_Q     SiLU(c) of the AVX route (c / (EXP8(0 - c) + 1)), rounded to
//              Q8_0 per 32 outputs into yq [m][rows], ys [m][rows/32]
//   GLU        rows paired (grx_glu_row): y [m][rows/2] = a * sigmoid(b)
//              (the K-split kernel and the one-row GEMV only)
//
// A wave computes 16 activation rows x 16*NS weight rows (NS 16x16 MFMA
// tiles sharing the A fragment; NS of 1 or 2 give small products more
// waves); a workgroup stacks four waves along the activation rows.  The
// blocks are walked U at a time with two register sets: the loads of the
// next U blocks are in flight while the current ones fold.
template <int EPI, int NS, int U>
__global__ __launch_bounds__(256) void gemm_q8_mfma_kernel(const int8_t *__restrict__ qs,
                                                           const uint16_t *__restrict__ ds, int rows, int nb,
                                                           const int8_t *__restrict__ xq,
                                                           const float *__restrict__ xs, int m,
                                                           const float *__restrict__ bias, float *__restrict__ y,
                                                           int ldc, float scale, int8_t *__restrict__ yq,
                                                           float *__restrict__ ys) {
    static_assert(NS == 1 || NS == 2 || NS == 4, "a 64-row weight tile splits into 1, 2 or 4 column groups");
    constexpr int kGroups = 4 / NS;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tile = blockIdx.y / kGroups;                // weight rows 64*tile ..
    const int sg = (blockIdx.y % kGroups) * NS;           // first 16-row group of the tile
    const int m0 = blockIdx.x * 64 + wave * 16;           // activation rows m0 .. m0+15
    const int K = nb * GRX_QK;
    const int li = lane & 15, lk = lane >> 4;             // fragment row/column, k group of 8

    // A fragment: row m0+li, bytes 8*lk..8*lk+7 of each block
    const int arow = m0 + li;
    const bool arow_ok = arow < m;
    const int8_t *ap = xq + (size_t)(arow_ok ? arow : 0) * K + 8 * lk;
    // B fragments: weight row 16*(sg+s)+li of the tile, bytes 8*lk..: half lk/2, offset 8*(lk&1)
    const int8_t *bp = qs + (size_t)tile * nb * 2048 + (lk >> 1) * 1024 + (16 * sg + li) * 16 + 8 * (lk & 1);
    const uint16_t *dp = ds + (size_t)tile * nb * 64 + 16 * sg + li;
    // D layout: lane holds column li, rows 4*lk + r
    int drow[4];
    bool drow_ok[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        drow[r] = m0 + 4 * lk + r;
        drow_ok[r] = drow[r] < m;
    }
    const float *sp[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) sp[r] = xs + (size_t)(drow_ok[r] ? drow[r] : 0) * nb;

    float c[NS][4];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        const int n = tile * 64 + 16 * (sg + s) + li;
        const float bv = (bias != nullptr && n < rows) ? bias[n] : 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) c[s][r] = bv;
    }

    struct Set {
        long av[U], bv[U][NS];
        uint32_t dh[U][NS];
        float da[U][4];
    };
    // activation scales four blocks per 16-byte load when the rows allow it
    // (nb % 4 == 0, whole groups of U): one load per four blocks per row
    const bool da4 = (nb & 3) == 0;
    auto load = [&](Set &S, int b0, int cnt) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (u >= cnt) break;
            const int b = b0 + u;
            S.av[u] = arow_ok ? *reinterpret_cast<const long *>(ap + (size_t)b * GRX_QK) : 0l;
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                S.bv[u][s] = *reinterpret_cast<const long *>(bp + (size_t)b * 2048 + s * 256);
                S.dh[u][s] = dp[(size_t)b * 64 + 16 * s];
            }
        }
        if (U % 4 == 0 && cnt == U && da4) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int q = 0; q < U / 4; ++q) {
                    const float4 v = *reinterpret_cast<const float4 *>(sp[r] + b0 + 4 * q);
                    S.da[4 * q + 0][r] = v.x;
                    S.da[4 * q + 1][r] = v.y;
                    S.da[4 * q + 2][r] = v.z;
                    S.da[4 * q + 3][r] = v.w;
                }
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (u >= cnt) break;
#pragma unroll
                for (int r = 0; r < 4; ++r) S.da[u][r] = sp[r][b0 + u];
            }
        }
    };
    // per block in order: s = the int32 dot (one MFMA per 16x16 tile, K 32 =
    // one Q8_0 block), then c = fma(f32(s) * dw, da, c)
    auto fold = [&](const Set &S, int cnt) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (u >= cnt) break;
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                v4i d = {0, 0, 0, 0};
                d = __builtin_amdgcn_mfma_i32_16x16x32_i8(S.av[u], S.bv[u][s], d, 0, 0, 0);
                const float dw = grx_f16_to_f32((uint16_t)S.dh[u][s]);
#pragma unroll
                for (int r = 0; r < 4; ++r) c[s][r] = __fmaf_rn(__fmul_rn((float)d[r], dw), S.da[u][r], c[s][r]);
            }
        }
    };
    Set s0, s1;
    int b = 0;
    if (nb >= U) load(s0, 0, U);
    // whole groups of U with the next group's loads in flight
    while (b + 2 * U <= nb) {
        load(s1, b + U, U);
        fold(s0, U);
        b += U;
        if (b + 2 * U <= nb) {
            load(s0, b + U, U);
            fold(s1, U);
            b += U;
        } else {
            fold(s1, U);
            b += U;
            if (b + U <= nb) {  // one more whole group
                load(s0, b, U);
                fold(s0, U);
                b += U;
            }
            goto tail;
        }
    }
    if (b + U <= nb) {  // a last whole group, loaded already
        fold(s0, U);
        b += U;
    }
tail:
    for (; b < nb; ++b) {  // the remaining blocks one at a time
        Set t;
        load(t, b, 1);
        fold(t, 1);
    }

    if constexpr (EPI == GRX_GEMM_SILU_Q) {
        // The wave's columns are whole Q8_0 blocks (NS even): block j holds
        // columns 16*(2j) + li and 16*(2j+1) + li of the 16 lanes sharing lk,
        // so a row's block maximum is four xor-shuffles within those lanes.
        static_assert(NS % 2 == 0, "rounded output needs whole 32-column blocks per wave");
        const int nr = rows / GRX_QK;
#pragma unroll
        for (int j = 0; j < NS / 2; ++j) {
            const int n0 = tile * 64 + 16 * sg + 32 * j;
            const bool col_ok = n0 < rows;  // rows % 32 == 0: whole blocks
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v[2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const float x = c[2 * j + h][r];
                    v[h] = __fdiv_rn(x, __fadd_rn(grx_exp8(__fsub_rn(0.0f, x)), 1.0f));
                }
                const float a0 = fabsf(v[0]), a1 = fabsf(v[1]);
                float amax = a0 > 0.0f ? a0 : 0.0f;
                amax = a1 > amax ? a1 : amax;
#pragma unroll
                for (int o = 8; o > 0; o >>= 1) {
                    const float t = __shfl_xor(amax, o, 16);
                    amax = t > amax ? t : amax;
                }
                const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
                if (col_ok && drow_ok[r]) {
                    int8_t *qrow = yq + (size_t)drow[r] * rows + n0;
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        float q = rintf(__fmul_rn(v[h], id));
                        q = fminf(fmaxf(q, -128.0f), 127.0f);
                        qrow[16 * h + li] = (int8_t)(int)q;
                    }
                    if (li == 0) ys[(size_t)drow[r] * nr + n0 / GRX_QK] = __fmul_rn(amax, grx_bits_f32(0x3c010204u));
                }
            }
        }
    } else {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int n = tile * 64 + 16 * (sg + s) + li;
            if (n >= rows) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (!drow_ok[r]) continue;
                float *yp = y + (size_t)drow[r] * ldc + n;
                if constexpr (EPI == GRX_GEMM_STORE) *yp = c[s][r];
                if constexpr (EPI == GRX_GEMM_ADD) *yp = __fadd_rn(*yp, c[s][r]);
                if constexpr (EPI == GRX_GEMM_AXPY_HALF) *yp = __fmaf_rn(0.5f, c[s][r], *yp);
                if constexpr (EPI == GRX_GEMM_SCALE) *yp = __fmul_rn(c[s][r], scale);
            }
        }
    }
}

// The product for fewer rows (m < 256: one utterance's encoder rows, a
// streaming chunk): a workgroup owns one output tile of 16 activation rows x
// 16*NS weight rows and splits the weight's blocks among its ks waves, KB
// consecutive blocks each, so that even a 1024-row product puts thousands of
// waves on the device and every wave issues all of its loads at once (the
// whole-K register walk above waits out one memory latency per U blocks).
// Each wave takes its blocks' int32 dots on the matrix cores and forms
// t_b = f32(s_b) * dw_b for them (order-free); the ordered chain
// c = fma(t_b, da_b, c) then runs wave after wave: wave 0 from the bias over
// blocks 0..KB-1, and each next wave from the c the previous one left in
// LDS, so every output sees the blocks in order, as in the other kernels.
// The tiles are numbered so that the workgroups of one weight column group
// (the row groups of the activations) land on one XCD and share its L2:
// workgroup i runs on XCD i % 8.
// Waves a workgroup of the K-split kernel may have: 16 where a wave's
// registers fit four waves a SIMD (16-column tiles of up to 8 blocks, 32-
// column tiles of 4), else 8.
constexpr int ks_max_waves(int ns, int kb) { return (ns == 1 && kb <= 8) || (ns == 2 && kb == 4) ? 16 : 8; }

template <int EPI, int NS, int KB>
__global__ __launch_bounds__(64 * ks_max_waves(NS, KB)) void gemm_q8_ks_kernel(
    const int8_t *__restrict__ qs, const uint16_t *__restrict__ ds, int rows, int nb, const int8_t *__restrict__ xq,
    const float *__restrict__ xs, int m, const float *__restrict__ bias, float *__restrict__ y, int ldc, float scale,
    int8_t *__restrict__ yq, float *__restrict__ ys, int ncg, int nrf, int da4, int bbeg, int bend,
    const float *init, int ldi) {
    static_assert(NS == 1 || NS == 2, "16 or 32 weight rows per tile");
    static_assert(KB % 4 == 0, "blocks per wave in whole groups of four");
    __shared__ float cx[2][NS * 4][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ks = __builtin_amdgcn_readfirstlane(blockDim.x >> 6);
    const int gi = blockIdx.x, xcd = gi & 7, slot = gi >> 3;
    const int rf = slot % nrf, cg = (slot / nrf) * 8 + xcd;
    if (cg >= ncg) return;  // the whole workgroup: no barrier is skipped
    const int K = nb * GRX_QK;
    const int li = lane & 15, lk = lane >> 4;
    const int n0 = cg * 16 * NS;                          // first weight row of the tile
    const int tile = n0 >> 6, sub = n0 & 63;              // 64-row weight tile, row offset in it
    // blocks bbeg..bend-1 of the nb (a run of them when the chain is carried
    // through init); the chain starts from init[row][col] when given, else
    // from the bias
    const int b0 = bbeg + wave * KB;
    const int nbw = min(KB, bend - b0);                   // this wave's blocks (>= 1)

    // A: activation row 16*rf+li (clamped: rows past m are computed, never
    // stored), bytes 8*lk.. of each block
    const int arow = min(16 * rf + li, m - 1);
    const int8_t *ap = xq + (size_t)arow * K + 8 * lk;
    const int8_t *bp = qs + (size_t)tile * nb * 2048 + (lk >> 1) * 1024 + (sub + li) * 16 + 8 * (lk & 1);
    const uint16_t *dp = ds + (size_t)tile * nb * 64 + sub + li;
    // D: lane holds weight row n0+16s+li, activation rows 16*rf+4*lk+r
    int drow[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) drow[r] = 16 * rf + 4 * lk + r;
    const float *sp[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) sp[r] = xs + (size_t)min(drow[r], m - 1) * nb;

    // every load of the wave's blocks in flight at once (the last wave's
    // block indices past nb are clamped and their results never used)
    long av[KB], bv[KB][NS];
    uint16_t dh[KB][NS];
    float da[KB][4];
#pragma unroll
    for (int u = 0; u < KB; ++u) {
        const int b = min(b0 + u, bend - 1);
        av[u] = *reinterpret_cast<const long *>(ap + (size_t)b * GRX_QK);
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            bv[u][s] = *reinterpret_cast<const long *>(bp + (size_t)b * 2048 + s * 256);
            dh[u][s] = dp[(size_t)b * 64 + 16 * s];
        }
    }
    if (da4) {  // nb % 4 == 0 and xs 16-byte aligned: four blocks per load
#pragma unroll
        for (int q = 0; q < KB / 4; ++q) {
            const int b = min(b0 + 4 * q, bend - 4);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float4 v = *reinterpret_cast<const float4 *>(sp[r] + b);
                da[4 * q + 0][r] = v.x;
                da[4 * q + 1][r] = v.y;
                da[4 * q + 2][r] = v.z;
                da[4 * q + 3][r] = v.w;
            }
        }
    } else {
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            const int b = min(b0 + u, bend - 1);
#pragma unroll
            for (int r = 0; r < 4; ++r) da[u][r] = sp[r][b];
        }
    }
    // the block dots and their scaled forms t = f32(s) * dw
    float t[KB][NS][4];
#pragma unroll
    for (int u = 0; u < KB; ++u) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            v4i d = {0, 0, 0, 0};
            d = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[u], bv[u][s], d, 0, 0, 0);
            const float dw = grx_f16_to_f32(dh[u][s]);
#pragma unroll
            for (int r = 0; r < 4; ++r) t[u][s][r] = __fmul_rn((float)d[r], dw);
        }
    }

    // the ordered chain, one wave after another
    float c[NS][4];
    for (int p = 0; p < ks; ++p) {
        if (wave == p) {
            if (p == 0 && init != nullptr) {
#pragma unroll
                for (int s = 0; s < NS; ++s) {
                    const int n = min(n0 + 16 * s + li, rows - 1);
#pragma unroll
                    for (int r = 0; r < 4; ++r) c[s][r] = init[(size_t)min(drow[r], m - 1) * ldi + n];
                }
            } else if (p == 0) {
#pragma unroll
                for (int s = 0; s < NS; ++s) {
                    const int n = n0 + 16 * s + li;
                    const float bv0 = (bias != nullptr && n < rows) ? bias[n] : 0.0f;
#pragma unroll
                    for (int r = 0; r < 4; ++r) c[s][r] = bv0;
                }
            } else {
#pragma unroll
                for (int s = 0; s < NS; ++s)
#pragma unroll
                    for (int r = 0; r < 4; ++r) c[s][r] = cx[(p - 1) & 1][4 * s + r][lane];
            }
            if (nbw == KB) {
#pragma unroll
                for (int u = 0; u < KB; ++u)
#pragma unroll
                    for (int s = 0; s < NS; ++s)
#pragma unroll
                        for (int r = 0; r < 4; ++r) c[s][r] = __fmaf_rn(t[u][s][r], da[u][r], c[s][r]);
            } else {
#pragma unroll
                for (int u = 0; u < KB; ++u) {
                    if (u < nbw) {
#pragma unroll
                        for (int s = 0; s < NS; ++s)
#pragma unroll
                            for (int r = 0; r < 4; ++r) c[s][r] = __fmaf_rn(t[u][s][r], da[u][r], c[s][r]);
                    }
                }
            }
            if (p + 1 < ks) {
#pragma unroll
                for (int s = 0; s < NS; ++s)
#pragma unroll
                    for (int r = 0; r < 4; ++r) cx[p & 1][4 * s + r][lane] = c[s][r];
            }
        }
        if (p + 1 < ks) __syncthreads();
    }
    if (wave != ks - 1) return;

    if constexpr (EPI == GRX_GEMM_SILU_Q) {
        // the tile's 32 columns are one Q8_0 block (rows % 32 == 0): a row's
        // block maximum is four xor-shuffles among the 16 lanes sharing lk
        static_assert(NS == 2, "rounded output needs whole 32-column blocks per tile");
        const int nr = rows / GRX_QK;
        const bool col_ok = n0 < rows;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float v[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float x = c[h][r];
                v[h] = __fdiv_rn(x, __fadd_rn(grx_exp8(__fsub_rn(0.0f, x)), 1.0f));
            }
            const float a0 = fabsf(v[0]), a1 = fabsf(v[1]);
            float amax = a0 > 0.0f ? a0 : 0.0f;
            amax = a1 > amax ? a1 : amax;
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) {
                const float tt = __shfl_xor(amax, o, 16);
                amax = tt > amax ? tt : amax;
            }
            const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
            if (col_ok && drow[r] < m) {
                int8_t *qrow = yq + (size_t)drow[r] * rows + n0;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    float q = rintf(__fmul_rn(v[h], id));
                    q = fminf(fmaxf(q, -128.0f), 127.0f);
                    qrow[16 * h + li] = (int8_t)(int)q;
                }
                if (li == 0) ys[(size_t)drow[r] * nr + n0 / GRX_QK] = __fmul_rn(amax, grx_bits_f32(0x3c010204u));
            }
        }
    } else {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int n = n0 + 16 * s + li;
            if (n >= rows) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (drow[r] >= m) continue;
                float *yp = y + (size_t)drow[r] * ldc + n;
                if constexpr (EPI == GRX_GEMM_STORE) *yp = c[s][r];
                if constexpr (EPI == GRX_GEMM_ADD) *yp = __fadd_rn(*yp, c[s][r]);
                if constexpr (EPI == GRX_GEMM_AXPY_HALF) *yp = __fmaf_rn(0.5f, c[s][r], *yp);
                if constexpr (EPI == GRX_GEMM_SCALE) *yp = __fmul_rn(c[s][r], scale);
            }
        }
    }
}

// The K-split product with its activations staged through LDS, for up to
// 255 rows: the same tiles, waves and ordered chain as gemm_q8_ks_kernel,
// but each wave copies its 16 activation rows x KB blocks into LDS with
// 16-byte loads (a row's KB*32 bytes in whole cache lines, where a fragment
// load touches 16 rows' lines for 32 bytes each) and the activation scales
// with one more, and the matrix cores take the weights as the A operand and
// the activations as B.  A lane then holds four consecutive weight rows of
// one activation row: its chain needs one activation scale per block (a
// 4-byte LDS read), its weight scales come as one 8-byte load per block,
// and its outputs are four consecutive floats of one output row.  Offsets
// from the (uniform) operand bases are 32-bit.
// Bytes of LDS per wave: 16 rows of KB*32 bytes, 16 apart beyond that (the
// fragment reads of 16 rows fall in different banks), then the scales as
// [block][row].
constexpr int kss_row(int kb) { return kb * 32 + 16; }
// The scales as [block][row], blocks kSdStride floats apart: a lane (row i,
// scale quad q) stores blocks 4q..4q+3, so with a stride of 20 the four
// lanes of a row write 16 banks apart (with 16 they shared a bank).
constexpr int kSdStride = 20;
constexpr int kss_bytes(int kb) { return 16 * kss_row(kb) + kSdStride * kb * 4; }

// The K-split kernel's fused parts: PRO 1 builds the staged activations
// from x rows by LayerNorm and rounding, PRO 2 by two LayerNorms with the
// first stored to x_out; the GLU epilogue's valid rows; a ring copy of the
// outputs.
struct KsFuse {
    const float *x;
    int lda;
    const float *lw, *lb, *lw2, *lb2;
    float *x_out;
    const int *lens;
    int T;
    RingCopy ring;
};
constexpr int kKsProPieces = 4;  // a fused prologue's rows: at most 4 float4 pieces a lane (1024 values)

// A fused prologue's product runs its chain on at most kKsProWaves waves,
// and its workgroup has a wave for each row of the 16-row group besides
// (kKsProLnWaves in all): each row's LayerNorm (float64 sums and their
// checks, one wave's dependent chain) is one wave's, the waves past the
// chain's only normalizing their rows.
constexpr int kKsProWaves = 8;
constexpr int kKsProLnWaves = 16;
template <int EPI, int NS, int KB, int PRO = 0>
__global__ __launch_bounds__(64 * (PRO != 0 ? kKsProLnWaves : ks_max_waves(NS, KB)), PRO != 0 ? 1 : 4) void
gemm_q8_kss_kernel(
    const int8_t *__restrict__ qs, const uint16_t *__restrict__ ds, int rows, int nb, const int8_t *__restrict__ xq,
    const float *__restrict__ xs, int m, const float *__restrict__ bias, float *__restrict__ y, int ldc, float scale,
    int8_t *__restrict__ yq, float *__restrict__ ys, int ncg, int nrf, int bbeg, int bend, const float *init,
    int ldi, const KsFuse f) {
    static_assert(NS == 1 || NS == 2, "16 or 32 weight rows per tile");
    static_assert(KB % 4 == 0, "blocks per wave in whole groups of four");
    static_assert(EPI != GRX_GEMM_GLU || NS == 2, "GLU pairs take 32-row tiles");
    __shared__ float cx[2][NS * 4][64];
    extern __shared__ __align__(16) int8_t kss_stage[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // nw waves, the first ks of them the chain's (a fused prologue's
    // workgroup has more: they only normalize rows, and pass the barriers)
    const int nw = __builtin_amdgcn_readfirstlane(blockDim.x >> 6);
    const int ks = PRO != 0 ? (bend - bbeg + KB - 1) / KB : nw;
    const bool chain = PRO == 0 || wave < ks;  // one of the chain's waves
    const int gi = blockIdx.x, xcd = gi & 7, slot = gi >> 3;
    const int rf = slot % nrf, cg = (slot / nrf) * 8 + xcd;
    if (cg >= ncg) return;  // the whole workgroup: no barrier is skipped
    const unsigned K = (unsigned)nb * GRX_QK;
    const int li = lane & 15, lk = lane >> 4;
    const int n0 = cg * 16 * NS;              // first weight row of the tile
    const int tile = n0 >> 6, sub = n0 & 63;  // 64-row weight tile, row offset in it
    const int b0 = bbeg + wave * KB;
    const int nbw = min(KB, bend - b0);       // this wave's blocks (>= 1)
    const int8_t *wq = qs + (size_t)tile * nb * 2048;
    const uint16_t *wd = ds + (size_t)tile * nb * 64;
    // A: weight row n0+16s+li, bytes 8*lk.. of each block; the lane's D rows
    // are n0+16s+4*lk .. +3, whose four weight scales are 8 contiguous bytes
    const unsigned qoff = (unsigned)((lk >> 1) * 1024 + (sub + li) * 16 + 8 * (lk & 1));
    const int arow = 16 * rf + li;            // the lane's activation row (B column)
    constexpr bool kResid = (EPI == GRX_GEMM_ADD || EPI == GRX_GEMM_AXPY_HALF) && NS == 1;
    constexpr int RS = kss_row(KB);
    int8_t *sa = kss_stage + wave * kss_bytes(KB);
    float *sd = reinterpret_cast<float *>(sa + 16 * RS);

    // the chain's start (wave 0: a carried chain's init, else the bias) is
    // loaded first, ahead of the operands, so the first link of the chain
    // does not wait on memory
    float cz[NS][4];
    if (wave == 0) {
        const int ar = min(arow, m - 1);
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int n = n0 + 16 * s + 4 * lk + r;
                cz[s][r] = init != nullptr ? init[(size_t)ar * ldi + min(n, rows - 1)]
                                           : ((bias != nullptr && n < rows) ? bias[n] : 0.0f);
            }
    }

    // every load of the wave's blocks in flight at once (block indices past
    // bend are clamped and their results never used; rows past m likewise)
    constexpr int NA = PRO == 0 ? KB / 2 : 1;  // 16-byte loads of the 16 rows x KB blocks
    int4 ra[NA];
    constexpr int DQ = KB / 4;  // float4s of scales per row
    float4 rd = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (PRO == 0) {
#pragma unroll
        for (int j = 0; j < NA; ++j) {
            const int e = j * 64 + lane, i = e / (2 * KB), pc = e % (2 * KB);
            const unsigned row = (unsigned)min(16 * rf + i, m - 1), b = (unsigned)min(b0 + pc / 2, bend - 1);
            ra[j] = *reinterpret_cast<const int4 *>(xq + (row * K + b * GRX_QK + (pc & 1) * 16));
        }
        if (lane < 16 * DQ) {
            const int i = lane / DQ, q = lane % DQ;
            const unsigned row = (unsigned)min(16 * rf + i, m - 1), b = (unsigned)min(b0 + 4 * q, bend - 4);
            rd = *reinterpret_cast<const float4 *>(xs + (row * (unsigned)nb + b));
        }
    }
    // a fused prologue's row (row `wave` of the group) and the LayerNorm
    // gains and biases, issued ahead of the weights so that the LayerNorm
    // waits on these loads only (a row past m is clamped to row m - 1 and
    // never staged)
    constexpr int NPP = PRO == 0 ? 1 : kKsProPieces;
    const int npc = (int)(K / 4);
    float4 xv[NPP], wv[NPP], bw[NPP];
    auto load_gains = [&](const float *lw, const float *lb) {
#pragma unroll
        for (int j = 0; j < NPP; ++j) {
            const int P = min(j * 64 + lane, npc - 1);
            wv[j] = reinterpret_cast<const float4 *>(lw)[P];
            bw[j] = reinterpret_cast<const float4 *>(lb)[P];
        }
    };
    if constexpr (PRO != 0) {
        const float4 *x4 = reinterpret_cast<const float4 *>(f.x + (size_t)min(16 * rf + wave, m - 1) * f.lda);
#pragma unroll
        for (int j = 0; j < NPP; ++j) xv[j] = x4[min(j * 64 + lane, npc - 1)];
        load_gains(f.lw, f.lb);
        // keep the scheduler from hoisting the weight loads above these
        __builtin_amdgcn_sched_barrier(0);
    }
    long bv[KB][NS];
    uint2 wsq = make_uint2(0u, 0u);
    if (chain) {
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            const unsigned b = (unsigned)min(b0 + u, bend - 1);
#pragma unroll
            for (int s = 0; s < NS; ++s) bv[u][s] = *reinterpret_cast<const long *>(wq + (qoff + b * 2048 + s * 256));
        }
        // the weight scales in one load: lane q (< KB*NS*4) takes the four
        // rows n0+16s+4j.. of block u, q = (u*NS + s)*4 + j; the lanes that
        // need them fetch them from lane q with a cross-lane permute
        const int q = min(lane, KB * NS * 4 - 1), u = q / (4 * NS), s = (q >> 2) % NS, j = q & 3;
        const unsigned b = (unsigned)min(b0 + u, bend - 1);
        wsq = *reinterpret_cast<const uint2 *>(reinterpret_cast<const char *>(wd) + 2 * (sub + 16 * s + 4 * j + b * 64));
    }
    // the epilogue's residual (the last wave; each element of y is read and
    // written by one lane only), loaded last, long before it is used (16
    // columns a wave: 32 would not leave the registers for four waves a SIMD)
    float yr[NS][4];
    if (kResid && wave == ks - 1 && arow < m) {
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int n = n0 + 16 * s + 4 * lk + r;
                yr[s][r] = n < rows ? y[(size_t)arow * ldc + n] : 0.0f;
            }
    }
    // the ring copy's head (the stream's control word), read early
    const int rhead = f.ring.p != nullptr ? ring_head(f.ring) : 0;
    if constexpr (PRO == 0) {
#pragma unroll
        for (int j = 0; j < NA; ++j) {
            const int e = j * 64 + lane, i = e / (2 * KB), pc = e % (2 * KB);
            *reinterpret_cast<int4 *>(sa + i * RS + pc * 16) = ra[j];
        }
        if (lane < 16 * DQ) {
            const int i = lane / DQ, q = lane % DQ;
            sd[(4 * q + 0) * kSdStride + i] = rd.x;
            sd[(4 * q + 1) * kSdStride + i] = rd.y;
            sd[(4 * q + 2) * kSdStride + i] = rd.z;
            sd[(4 * q + 3) * kSdStride + i] = rd.w;
        }
    } else {
        // the fused prologue (one run of all nb blocks, K <= 1024): wave w
        // takes row w of the 16-row group (the launch gives the workgroup a
        // wave for each row), held as NP float4 pieces a lane,
        // LayerNorm'd by wave_ln32 (kern.LayerNorm, internal/kern/mathx.go:
        // 55-75), and rounds each 32-value block (8 pieces in 8 lanes;
        // quantU8, q8int.go:88-105) into the stage of the wave that owns the
        // block.  Rows past m are not staged: their products are never
        // stored.
        constexpr int NP = kKsProPieces;
        auto one_row = [&](int i) {
            wave_ln32<NP>(xv, wv, bw, npc, lane);
            if constexpr (PRO == 2) {
                // a block's norm_out (conformer/encoder.go:426), kept by the
                // first column group, then the next block's LayerNorm (its
                // gains in the first's registers, loaded while its
                // statistics form)
                load_gains(f.lw2, f.lb2);
                if (cg == 0) {
                    float4 *xo = reinterpret_cast<float4 *>(f.x_out + (size_t)(16 * rf + i) * f.lda);
#pragma unroll
                    for (int j = 0; j < NP; ++j)
                        if (j * 64 + lane < npc) xo[j * 64 + lane] = xv[j];
                }
                wave_ln32<NP>(xv, wv, bw, npc, lane);
            }
#pragma unroll
            for (int j = 0; j < NP; ++j) {
                const float4 v = xv[j];
                float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
                for (int o = 4; o > 0; o >>= 1) {
                    const float tt = __shfl_xor(amax, o, 8);
                    amax = tt > amax ? tt : amax;
                }
                const int P = j * 64 + lane;
                if (P >= npc) continue;
                const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
                auto q1 = [&](float x) {
                    float tq = rintf(__fmul_rn(x, id));
                    tq = fminf(fmaxf(tq, -128.0f), 127.0f);
                    return (uint32_t)(uint8_t)(int8_t)(int)tq;
                };
                const uint32_t pk = q1(v.x) | q1(v.y) << 8 | q1(v.z) << 16 | q1(v.w) << 24;
                const int blk = P >> 3, ow = blk / KB, u = blk - ow * KB;
                int8_t *so = kss_stage + ow * kss_bytes(KB);
                *reinterpret_cast<uint32_t *>(so + i * RS + u * GRX_QK + 4 * (P & 7)) = pk;
                if ((P & 7) == 0)
                    reinterpret_cast<float *>(so + 16 * RS)[u * kSdStride + i] = __fmul_rn(amax, grx_bits_f32(0x3c010204u));
            }
        };
        if (wave < 16 && 16 * rf + wave < m) one_row(wave);
    }
    __syncthreads();

    // the block dots (weight rows 4*lk+r of the 16, activation row li) and
    // their scaled forms t = f32(s) * dw (the chain's waves only)
    float t[KB][NS][4];
    if (chain) {
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            const long a = *reinterpret_cast<const long *>(sa + li * RS + u * GRX_QK + 8 * lk);
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                v4i d = {0, 0, 0, 0};
                d = __builtin_amdgcn_mfma_i32_16x16x32_i8(bv[u][s], a, d, 0, 0, 0);
                const int src = ((u * NS + s) * 4 + lk) * 4;
                const uint32_t h[2] = {(uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)wsq.x),
                                       (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)wsq.y)};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float dw = grx_f16_to_f32((uint16_t)(h[r >> 1] >> (16 * (r & 1))));
                    t[u][s][r] = __fmul_rn((float)d[r], dw);
                }
            }
        }
    }

    // the chain's activation scales, read before the wave's turn comes (16
    // columns a wave; with 32 the registers go to the products, and each
    // read is followed by eight links rather than four)
    constexpr bool kHoist = NS == 1;
    float dav[kHoist ? KB : 1];
    if constexpr (kHoist) {
#pragma unroll
        for (int u = 0; u < KB; ++u) dav[u] = chain ? sd[u * kSdStride + li] : 0.0f;
    }

    // the ordered chain, one wave after another
    float c[NS][4];
    for (int p = 0; p < ks; ++p) {
        if (wave == p) {
            if (p == 0) {
#pragma unroll
                for (int s = 0; s < NS; ++s)
#pragma unroll
                    for (int r = 0; r < 4; ++r) c[s][r] = cz[s][r];
            } else {
#pragma unroll
                for (int s = 0; s < NS; ++s)
#pragma unroll
                    for (int r = 0; r < 4; ++r) c[s][r] = cx[(p - 1) & 1][4 * s + r][lane];
            }
            if (nbw == KB) {
#pragma unroll
                for (int u = 0; u < KB; ++u) {
                    const float da = kHoist ? dav[kHoist ? u : 0] : sd[u * kSdStride + li];
#pragma unroll
                    for (int s = 0; s < NS; ++s)
#pragma unroll
                        for (int r = 0; r < 4; ++r) c[s][r] = __fmaf_rn(t[u][s][r], da, c[s][r]);
                }
            } else {
#pragma unroll
                for (int u = 0; u < KB; ++u) {
                    if (u < nbw) {
                        const float da = kHoist ? dav[kHoist ? u : 0] : sd[u * kSdStride + li];
#pragma unroll
                        for (int s = 0; s < NS; ++s)
#pragma unroll
                            for (int r = 0; r < 4; ++r) c[s][r] = __fmaf_rn(t[u][s][r], da, c[s][r]);
                    }
                }
            }
            if (p + 1 < ks) {
#pragma unroll
                for (int s = 0; s < NS; ++s)
#pragma unroll
                    for (int r = 0; r < 4; ++r) cx[p & 1][4 * s + r][lane] = c[s][r];
            }
        }
        if (p + 1 < ks) __syncthreads();
    }
    if (wave != ks - 1) return;

    if constexpr (EPI == GRX_GEMM_SILU_Q) {
        // the tile's 32 columns are one Q8_0 block of the activation row
        // (rows % 32 == 0), spread over the four lanes li, li+16, li+32,
        // li+48: their block maximum is two xor-shuffles
        static_assert(NS == 2, "rounded output needs whole 32-column blocks per tile");
        const int nr = rows / GRX_QK;
        float v[2][4];
        float amax = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float x = c[h][r];
                v[h][r] = __fdiv_rn(x, __fadd_rn(grx_exp8(__fsub_rn(0.0f, x)), 1.0f));
                const float a = fabsf(v[h][r]);
                amax = a > amax ? a : amax;
            }
#pragma unroll
        for (int o = 16; o < 64; o <<= 1) {
            const float tt = __shfl_xor(amax, o);
            amax = tt > amax ? tt : amax;
        }
        const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
        if (n0 < rows && arow < m) {
            int8_t *qrow = yq + (size_t)arow * rows + n0;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                uint32_t pk = 0;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float q = rintf(__fmul_rn(v[h][r], id));
                    q = fminf(fmaxf(q, -128.0f), 127.0f);
                    pk |= (uint32_t)(uint8_t)(int8_t)(int)q << (8 * r);
                }
                *reinterpret_cast<uint32_t *>(qrow + 16 * h + 4 * lk) = pk;
            }
            if (lk == 0) ys[(size_t)arow * nr + n0 / GRX_QK] = __fmul_rn(amax, grx_bits_f32(0x3c010204u));
        }
    } else if constexpr (EPI == GRX_GEMM_GLU) {
        // the tile's rows n0..n0+15 are the a-rows of channels n0/2 ..
        // n0/2 + 15 and rows n0+16.. their b-rows: lane (li, lk) holds both
        // for channels n0/2 + 4 lk .. +3 of activation row arow
        if (arow >= m || n0 >= rows) return;
        const int sb = arow / f.T;
        const bool live = arow - sb * f.T < f.lens[sb];
        const int ch = (n0 >> 1) + 4 * lk;
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = live ? grx_glu_pair(c[0][r], c[1][r]) : 0.0f;
        *reinterpret_cast<float4 *>(y + (size_t)arow * ldc + ch) = make_float4(v[0], v[1], v[2], v[3]);
        if (f.ring.p != nullptr) {
            float *rr = ring_row(f.ring, rhead, arow);
#pragma unroll
            for (int r = 0; r < 4; ++r) ring_put(f.ring, rr, ch + r - f.ring.col0, v[r]);
        }
    } else {
        if (arow >= m) return;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int n = n0 + 16 * s + 4 * lk;
            float *yp = y + (size_t)arow * ldc + n;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (n + r >= rows) continue;
                if constexpr (EPI == GRX_GEMM_STORE) yp[r] = c[s][r];
                if constexpr (EPI == GRX_GEMM_ADD) yp[r] = __fadd_rn(kResid ? yr[s][r] : yp[r], c[s][r]);
                if constexpr (EPI == GRX_GEMM_AXPY_HALF) yp[r] = __fmaf_rn(0.5f, c[s][r], kResid ? yr[s][r] : yp[r]);
                if constexpr (EPI == GRX_GEMM_SCALE) yp[r] = __fmul_rn(c[s][r], scale);
            }
        }
        if constexpr (EPI == GRX_GEMM_STORE) {
            if (f.ring.p != nullptr) {
                float *rr = ring_row(f.ring, rhead, arow);
#pragma unroll
                for (int s = 0; s < NS; ++s)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int n = n0 + 16 * s + 4 * lk + r;
                        if (n < rows && n >= f.ring.col0) ring_put(f.ring, rr, n - f.ring.col0, c[s][r]);
                    }
            }
        }
    }
}

// The product for many activation rows: a workgroup of eight waves (2 x 4)
// computes 64 activation rows x 128 weight rows, each wave 32 x 32 (2 x 2
// MFMA tiles).  kLdsCB blocks at a time of the rounded activations, the two
// weight tiles, their scales and the activation scales are copied to LDS
// with 16-byte loads, double-buffered (the next blocks' loads are in flight
// while the current ones fold), so each activation row and weight row is
// read from L2 once per workgroup instead of once per wave.  Per output the
// fold is the same: c = fma(f32(s_b) * dw_b, da_b, c), blocks in order.
constexpr int kLdsCB = 4;
constexpr int kLdsThreads = 512;

template <int EPI>
__global__ __launch_bounds__(kLdsThreads) void gemm_q8_lds_kernel(const int8_t *__restrict__ qs,
                                                                  const uint16_t *__restrict__ ds, int rows, int nb,
                                                                  int tiles, const int8_t *__restrict__ xq,
                                                                  const float *__restrict__ xs, int m,
                                                                  const float *__restrict__ bias,
                                                                  float *__restrict__ y, int ldc, float scale,
                                                                  int8_t *__restrict__ yq, float *__restrict__ ys,
                                                                  const KsFuse fz) {
    // LDS per buffer: A [64 rows][CB][32] bytes, rows kAr apart (16 bytes of
    // padding: a fragment's 8-byte reads of 16 rows and a row's 16-byte
    // stores fall in distinct banks), B [CB][2 tiles][2 halves][64][16],
    // weight scales [CB][128] u16, activation scales [CB][64] f32
    constexpr int kAr = kLdsCB * 32 + 16;
    constexpr int kA = 64 * kAr, kB = kLdsCB * 2 * 2048, kD = kLdsCB * 128 * 2, kS = kLdsCB * 64 * 4;
    constexpr int kBuf = kA + kB + kD + kS;
    __shared__ __align__(16) uint8_t lds[2 * kBuf];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 2, wn = wave & 3;             // wave rows 32*wm.., columns 32*wn..
    const int mb = blockIdx.x * 64, t0 = blockIdx.y * 2;  // activation rows mb.., weight tiles t0, t0+1
    const int K = nb * GRX_QK;
    const int li = lane & 15, lk = lane >> 4;

    // ---- the copy of blocks [b0, b0+CB) into registers, then LDS
    // A: 64 rows x CB*32 bytes = 64 x (2*CB) 16-byte pieces (one per thread for CB 4)
    // B: 2 tiles x CB x 2048 bytes = 2*CB*128 pieces (two per thread)
    // dw: 2 tiles x CB x 128 bytes = 2*CB*8 pieces; da: 64 rows x CB floats (one piece per row)
    constexpr int kApc = 64 * 2 * kLdsCB, kBpc = 2 * kLdsCB * 128, kDpc = 2 * kLdsCB * 8;
    static_assert(kApc == kLdsThreads && kBpc == 2 * kLdsThreads, "copy split assumes CB 4 and 512 threads");
    uint4 ra, rb[2], rd;
    float4 rs;
    auto gload = [&](int b0) {
        {
            const int row = tid / (2 * kLdsCB), piece = tid % (2 * kLdsCB);
            const int gr = mb + row, bb = b0 + piece / 2;
            ra = (gr < m && bb < nb) ? *reinterpret_cast<const uint4 *>(xq + (size_t)gr * K + (size_t)bb * 32 + 16 * (piece & 1))
                                     : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int pc = tid + h * kLdsThreads;
            const int t = pc / (kLdsCB * 128), rem = pc % (kLdsCB * 128), u = rem / 128, off = rem % 128;
            const int tile = t0 + t, bb = b0 + u;
            rb[h] = (tile < tiles && bb < nb)
                        ? *reinterpret_cast<const uint4 *>(qs + ((size_t)tile * nb + bb) * 2048 + 16 * off)
                        : make_uint4(0, 0, 0, 0);
        }
        if (tid < kDpc) {
            const int t = tid / (kLdsCB * 8), rem = tid % (kLdsCB * 8), u = rem / 8, off = rem % 8;
            const int tile = t0 + t, bb = b0 + u;
            rd = (tile < tiles && bb < nb)
                     ? *reinterpret_cast<const uint4 *>(ds + ((size_t)tile * nb + bb) * 64 + 8 * off)
                     : make_uint4(0, 0, 0, 0);
        }
        if (tid >= kDpc && tid < kDpc + 64) {
            const int row = tid - kDpc, gr = mb + row;
#pragma unroll
            for (int u = 0; u < kLdsCB; ++u) {
                const float v = (gr < m && b0 + u < nb) ? xs[(size_t)gr * nb + b0 + u] : 0.0f;
                if (u == 0) rs.x = v;
                if (u == 1) rs.y = v;
                if (u == 2) rs.z = v;
                if (u == 3) rs.w = v;
            }
        }
    };
    auto lstore = [&](int buf) {
        uint8_t *base = lds + buf * kBuf;
        {
            const int row = tid / (2 * kLdsCB), piece = tid % (2 * kLdsCB);
            *reinterpret_cast<uint4 *>(base + row * kAr + 16 * piece) = ra;
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int pc = tid + h * kLdsThreads;
            const int t = pc / (kLdsCB * 128), rem = pc % (kLdsCB * 128), u = rem / 128, off = rem % 128;
            *reinterpret_cast<uint4 *>(base + kA + (u * 2 + t) * 2048 + 16 * off) = rb[h];
        }
        if (tid < kDpc) {
            const int t = tid / (kLdsCB * 8), rem = tid % (kLdsCB * 8), u = rem / 8, off = rem % 8;
            *reinterpret_cast<uint4 *>(base + kA + kB + (u * 128 + t * 64) * 2 + 16 * off) = rd;
        }
        if (tid >= kDpc && tid < kDpc + 64) {
            const int row = tid - kDpc;
            float *sa = reinterpret_cast<float *>(base + kA + kB + kD);
            sa[0 * 64 + row] = rs.x;
            sa[1 * 64 + row] = rs.y;
            sa[2 * 64 + row] = rs.z;
            sa[3 * 64 + row] = rs.w;
        }
    };

    float c[2][2][4];  // [row frag][column frag][r]
#pragma unroll
    for (int g = 0; g < 2; ++g) {
        const int n = t0 * 64 + 32 * wn + 16 * g + li;
        const float bv = (bias != nullptr && n < rows) ? bias[n] : 0.0f;
#pragma unroll
        for (int f = 0; f < 2; ++f)
#pragma unroll
            for (int r = 0; r < 4; ++r) c[f][g][r] = bv;
    }
    const int nsteps = (nb + kLdsCB - 1) / kLdsCB;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int st = 0; st < nsteps; ++st) {
        const int cur = st & 1;
        if (st + 1 < nsteps) gload((st + 1) * kLdsCB);
        const uint8_t *base = lds + cur * kBuf;
        const uint16_t *dwl = reinterpret_cast<const uint16_t *>(base + kA + kB);
        const float *dal = reinterpret_cast<const float *>(base + kA + kB + kD);
        const int ub = min(kLdsCB, nb - st * kLdsCB);
#pragma unroll
        for (int u = 0; u < kLdsCB; ++u) {
            if (u >= ub) break;
            long av[2], bv[2];
            float da[2][4], dw[2];
#pragma unroll
            for (int f = 0; f < 2; ++f) {
                const int row = 32 * wm + 16 * f + li;
                av[f] = *reinterpret_cast<const long *>(base + row * kAr + u * 32 + 8 * lk);
#pragma unroll
                for (int r = 0; r < 4; ++r) da[f][r] = dal[u * 64 + 32 * wm + 16 * f + 4 * lk + r];
            }
#pragma unroll
            for (int g = 0; g < 2; ++g) {
                const int col = 32 * wn + 16 * g + li;  // 0..127 across the two tiles
                const int t = col >> 6, cr = col & 63;
                bv[g] = *reinterpret_cast<const long *>(base + kA + (u * 2 + t) * 2048 + (lk >> 1) * 1024 + cr * 16 +
                                                        8 * (lk & 1));
                dw[g] = grx_f16_to_f32(dwl[u * 128 + col]);
            }
            // the block's four products issued together, then their folds:
            // no fold waits on a product issued just before it
            v4i d[2][2];
#pragma unroll
            for (int f = 0; f < 2; ++f)
#pragma unroll
                for (int g = 0; g < 2; ++g) {
                    const v4i z = {0, 0, 0, 0};
                    d[f][g] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[f], bv[g], z, 0, 0, 0);
                }
#pragma unroll
            for (int f = 0; f < 2; ++f)
#pragma unroll
                for (int g = 0; g < 2; ++g)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        c[f][g][r] = __fmaf_rn(__fmul_rn((float)d[f][g][r], dw[g]), da[f][r], c[f][g][r]);
        }
        if (st + 1 < nsteps) {
            lstore(cur ^ 1);
            __syncthreads();
        }
    }

#pragma unroll
    for (int f = 0; f < 2; ++f) {
        int drow[4];
        bool drow_ok[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            drow[r] = mb + 32 * wm + 16 * f + 4 * lk + r;
            drow_ok[r] = drow[r] < m;
        }
        if constexpr (EPI == GRX_GEMM_SILU_Q) {
            // the wave's 32 columns are one Q8_0 block (rows % 32 == 0)
            const int nr = rows / GRX_QK;
            const int n0 = t0 * 64 + 32 * wn;
            const bool col_ok = n0 < rows;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v[2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const float x = c[f][h][r];
                    v[h] = __fdiv_rn(x, __fadd_rn(grx_exp8(__fsub_rn(0.0f, x)), 1.0f));
                }
                const float a0 = fabsf(v[0]), a1 = fabsf(v[1]);
                float amax = a0 > 0.0f ? a0 : 0.0f;
                amax = a1 > amax ? a1 : amax;
#pragma unroll
                for (int o = 8; o > 0; o >>= 1) {
                    const float t = __shfl_xor(amax, o, 16);
                    amax = t > amax ? t : amax;
                }
                const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
                if (col_ok && drow_ok[r]) {
                    int8_t *qrow = yq + (size_t)drow[r] * rows + n0;
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        float q = rintf(__fmul_rn(v[h], id));
                        q = fminf(fmaxf(q, -128.0f), 127.0f);
                        qrow[16 * h + li] = (int8_t)(int)q;
                    }
                    if (li == 0) ys[(size_t)drow[r] * nr + n0 / GRX_QK] = __fmul_rn(amax, grx_bits_f32(0x3c010204u));
                }
            }
        } else if constexpr (EPI == GRX_GEMM_GLU) {
            // the wave's 32 columns are one pair group (grx_glu_row): its
            // 16 a-rows (g = 0) and their b-rows (g = 1) in the same lane,
            // channel n0/2 + li
            const int n0 = t0 * 64 + 32 * wn;
            if (n0 < rows) {
                const int rh = fz.ring.p != nullptr ? ring_head(fz.ring) : 0;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (!drow_ok[r]) continue;
                    const int sb = drow[r] / fz.T;
                    const float v = drow[r] - sb * fz.T < fz.lens[sb] ? grx_glu_pair(c[f][0][r], c[f][1][r]) : 0.0f;
                    const int ch = (n0 >> 1) + li;
                    y[(size_t)drow[r] * ldc + ch] = v;
                    if (fz.ring.p != nullptr) ring_put(fz.ring, ring_row(fz.ring, rh, drow[r]), ch - fz.ring.col0, v);
                }
            }
        } else {
            const int rh = (EPI == GRX_GEMM_STORE && fz.ring.p != nullptr) ? ring_head(fz.ring) : 0;
#pragma unroll
            for (int g = 0; g < 2; ++g) {
                const int n = t0 * 64 + 32 * wn + 16 * g + li;
                if (n >= rows) continue;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (!drow_ok[r]) continue;
                    float *yp = y + (size_t)drow[r] * ldc + n;
                    if constexpr (EPI == GRX_GEMM_STORE) {
                        *yp = c[f][g][r];
                        if (fz.ring.p != nullptr && n >= fz.ring.col0)
                            ring_put(fz.ring, ring_row(fz.ring, rh, drow[r]), n - fz.ring.col0, c[f][g][r]);
                    }
                    if constexpr (EPI == GRX_GEMM_ADD) *yp = __fadd_rn(*yp, c[f][g][r]);
                    if constexpr (EPI == GRX_GEMM_AXPY_HALF) *yp = __fmaf_rn(0.5f, c[f][g][r], *yp);
                    if constexpr (EPI == GRX_GEMM_SCALE) *yp = __fmul_rn(c[f][g][r], scale);
                }
            }
        }
    }
}

// Blocks per register set for each wave-tile width (swept on the device).
#ifndef GRX_GEMM_U1
#define GRX_GEMM_U1 8
#endif
#ifndef GRX_GEMM_U2
#define GRX_GEMM_U2 8
#endif
#ifndef GRX_GEMM_U4
#define GRX_GEMM_U4 4
#endif

// Column-group width for a product: enough waves to cover the device
// (16*NS weight rows per wave), NS = 4 once there are plenty.
int pick_ns(int m, int rows, int epi) {
    const int v = grx_tune(GRX_TUNE_GEMM_NS);
    if (v == 1 || v == 2 || v == 4) return (epi == GRX_GEMM_SILU_Q && v == 1) ? 2 : v;
    // (measured at 64 and 126 rows: two 16-column tiles per wave win from
    // about 384 of these on, e.g. 126 x 4096 x 1024 14.0 -> 10.0 us)
    const long waves4 = (long)grx_ceil_div(m, 16) * grx_ceil_div(rows, 64);
    int ns = waves4 >= 4096 ? 4 : (waves4 >= 384 ? 2 : 1);
    if (epi == GRX_GEMM_SILU_Q && ns == 1) ns = 2;
    return ns;
}

// The K-split kernel's tile width and blocks per wave.  Activations staged
// through LDS (sa; measured on MI355X at 126 rows): 32-column tiles of 8
// blocks for the wide short-K products (126 x 4096 x 1024 8.2 us against
// 8.9, 3072 x 1024 7.3 against 7.4), else 16-column tiles of 16 blocks
// (1024 x 4096 9.7 us, 1024 x 1024 5.1, 2048 x 1024 6.2); with one or two
// 16-row groups 8 blocks a wave up to 64 blocks (8 x 1280 x 1280 4.8 us
// against 5.0 for 4), 16 past that (14 x 1024 x 4096 8.0 against 9.1).
// Activations read straight from memory (16-byte alignment or whole
// groups of four blocks missing): 32-column tiles with 8 blocks per wave
// for K up to 2048 (126 x 1024 x 1024 7.7 -> 5.5 us, 14 x 4096 x 1024
// 5.9 -> 4.8 us), 16-column tiles with 16 blocks per wave past that
// (126 x 1024 x 4096 25 -> 19 us), and with one or two 16-row groups the
// fewest blocks per wave that fit a workgroup (8 x 1280 x 1280: 16 columns,
// 4 blocks a wave, 10 waves a workgroup).  The rounded SiLU output needs the
// 32-column tiles (whole Q8_0 blocks).  A carried chain runs in 16 waves x
// 8 blocks (8 x 1280 x 5120: 23.6 us on the GEMV, two runs here).  False
// when a workgroup of ks_max_waves waves cannot hold the weight's blocks.
bool pick_ks(int m, int nb, int rows, int epi, bool carry, bool sa, bool pro, int *ns, int *kb) {
    const bool pair = epi == GRX_GEMM_SILU_Q || epi == GRX_GEMM_GLU;  // whole 32-row tiles
    const bool few = grx_ceil_div(m, 16) <= 2 && !pair;
    int n, k;
    if (sa) {
        n = (pair || (!few && nb <= 2 * 8 * 4 && rows >= 3072)) ? 2 : 1;
        k = n == 2 ? 8 : 16;
        if (few) k = nb <= 64 ? 8 : 16;
    } else {
        n = (pair || (!few && nb <= 2 * 8 * 4)) ? 2 : 1;
        k = n == 2 ? 8 : 16;
        if (few) k = nb <= ks_max_waves(n, 4) * 4 ? 4 : 16;
    }
    if (few && carry && nb > ks_max_waves(n, 16) * 16) k = 8;
    // a fused prologue: 4 blocks a wave (its rows' LayerNorms take a wave
    // each besides; K <= 1024 fits kKsProWaves waves of the chain)
    if (pro) k = 4;
    const int tn = grx_tune(GRX_TUNE_GEMM_NS);
    if (tn == 1 || tn == 2) {
        n = pair ? 2 : tn;
        if (n == 2 && k > 8) k = 8;
    }
    const int tk = grx_tune(GRX_TUNE_GEMM_KB);
    if ((tk == 4 || tk == 8 || tk == 16) && !(n == 2 && tk == 16) && !pro) k = tk;
    if (n == 2 && k > 8) k = 8;
    if (nb > ks_max_waves(n, k) * k && !(carry && few)) return false;
    *ns = n;
    *kb = k;
    return true;
}

// Whether the staged-activation instantiation may take its LDS (asked once;
// more than 64 KB needs the attribute).
template <int EPI, int NS, int KB, int PRO>
bool ks_stage_ok() {
    static const bool ok = [] {
        const int need = ks_max_waves(NS, KB) * kss_bytes(KB);
        const bool r = need <= 64 * 1024 ||
                       hipFuncSetAttribute((const void *)gemm_q8_kss_kernel<EPI, NS, KB, PRO>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, need) == hipSuccess;
        (void)hipGetLastError();
        return r;
    }();
    return ok;
}

KsFuse ks_fuse(const GemmOut &o) {
    KsFuse f{};
    f.x = o.x;
    f.lda = o.lda;
    f.lw = o.ln_w;
    f.lb = o.ln_b;
    f.lw2 = o.ln_w2;
    f.lb2 = o.ln_b2;
    f.x_out = o.x_out;
    f.lens = o.lens;
    f.T = o.T > 0 ? o.T : 1;
    f.ring = o.ring;
    return f;
}

template <int EPI, int NS, int KB, bool SA, int PRO>
void launch_ks_run(hipStream_t st, const grx_weight *w, const int8_t *xq, const float *xs, int m, const float *bias,
                   float *y, int ldc, const GemmOut &o, int da4, int bbeg, int bend, const float *init) {
    // init (a carried chain) rows are w->rows apart
    const int ncg = grx_ceil_div(w->rows, 16 * NS), nrf = grx_ceil_div(m, 16);
    const int ks = grx_ceil_div(bend - bbeg, KB);
    const int groups = grx_ceil_div(ncg, 8) * 8 * nrf;
    // a fused prologue's workgroup: a wave for each row of a 16-row group
    // as well (those past the chain's ks only normalize rows)
    const int nw = PRO != 0 ? max(ks, min(16, m)) : ks;
    if constexpr (SA)
        gemm_q8_kss_kernel<EPI, NS, KB, PRO><<<groups, 64 * nw, (size_t)ks * kss_bytes(KB), st>>>(
            w->qs, w->ds, w->rows, w->nb, xq, xs, m, bias, y, ldc, o.scale, o.yq, o.ys, ncg, nrf, bbeg, bend, init,
            w->rows, ks_fuse(o));
    else
        gemm_q8_ks_kernel<EPI, NS, KB><<<groups, 64 * ks, 0, st>>>(w->qs, w->ds, w->rows, w->nb, xq, xs, m, bias, y,
                                                                   ldc, o.scale, o.yq, o.ys, ncg, nrf, da4, bbeg, bend,
                                                                   init, w->rows);
}

// The whole product: one launch, or (a carry buffer given, more blocks than
// a workgroup holds) runs of ks_max_waves * KB blocks, each continuing the
// chain the last one stored, the epilogue in the last.
template <int EPI, int NS, int KB, bool SA>
void launch_ks(hipStream_t st, const grx_weight *w, const int8_t *xq, const float *xs, int m, const float *bias,
               const GemmOut &o, int da4) {
    const int run = ks_max_waves(NS, KB) * KB;
    if (w->nb <= run || o.carry == nullptr) {
        launch_ks_run<EPI, NS, KB, SA, 0>(st, w, xq, xs, m, bias, o.y, o.ldc, o, da4, 0, w->nb, nullptr);
        return;
    }
    const float *init = nullptr;
    for (int b = 0; b < w->nb; b += run) {
        const int e = min(w->nb, b + run);
        if (e < w->nb) {
            launch_ks_run<GRX_GEMM_STORE, NS, KB, SA, 0>(st, w, xq, xs, m, bias, o.carry, w->rows, o, da4, b, e,
                                                         init);
            init = o.carry;
        } else {
            launch_ks_run<EPI, NS, KB, SA, 0>(st, w, xq, xs, m, bias, o.y, o.ldc, o, da4, b, e, init);
        }
    }
}

// SA when asked and possible: 16-byte aligned activations and scales, whole
// groups of four blocks, the LDS granted (for the carried runs' STORE
// instantiation too)
template <int EPI, int NS, int KB>
void launch_ks_sa(hipStream_t st, const grx_weight *w, const int8_t *xq, const float *xs, int m, const float *bias,
                  const GemmOut &o, int da4, bool sa) {
    if (sa && ks_stage_ok<EPI, NS, KB, 0>() && ks_stage_ok<GRX_GEMM_STORE, NS, KB, 0>())
        return launch_ks<EPI, NS, KB, true>(st, w, xq, xs, m, bias, o, da4);
    return launch_ks<EPI, NS, KB, false>(st, w, xq, xs, m, bias, o, da4);
}

template <int EPI>
void launch_ks_epi(hipStream_t st, const grx_weight *w, const int8_t *xq, const float *xs, int m, const float *bias,
                   const GemmOut &o, int ns, int kb, int da4, bool sa) {
    if constexpr (EPI != GRX_GEMM_SILU_Q) {
        if (ns == 1) {
            if (kb == 4) return launch_ks_sa<EPI, 1, 4>(st, w, xq, xs, m, bias, o, da4, sa);
            if (kb == 8) return launch_ks_sa<EPI, 1, 8>(st, w, xq, xs, m, bias, o, da4, sa);
            return launch_ks_sa<EPI, 1, 16>(st, w, xq, xs, m, bias, o, da4, sa);
        }
    }
    if (kb == 4) return launch_ks_sa<EPI, 2, 4>(st, w, xq, xs, m, bias, o, da4, sa);
    return launch_ks_sa<EPI, 2, 8>(st, w, xq, xs, m, bias, o, da4, sa);
}

// The fused forms (a prologue, GLU, a ring copy): the staged kernel in one
// run of blocks, 4 or 8 blocks a wave.
template <int EPI, int PRO>
void launch_ks_fused_pro(hipStream_t st, const grx_weight *w, const int8_t *xq, const float *xs, int m,
                         const float *bias, const GemmOut &o, int ns, int kb) {
    // pre-rounded activations come through xq/xs (PRO 0)
    const int8_t *q = PRO == 0 ? xq : nullptr;
    const float *sc = PRO == 0 ? xs : nullptr;
    auto go = [&](auto ns_tag, auto kb_tag) {
        constexpr int NS = decltype(ns_tag)::value, KB = decltype(kb_tag)::value;
        (void)ks_stage_ok<EPI, NS, KB, PRO>();
        launch_ks_run<EPI, NS, KB, true, PRO>(st, w, q, sc, m, bias, o.y, o.ldc, o, 1, 0, w->nb, nullptr);
    };
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using K4 = std::integral_constant<int, 4>;
    using K8 = std::integral_constant<int, 8>;
    using K16 = std::integral_constant<int, 16>;
    if constexpr (PRO != 0) {
        // a fused prologue: 4 blocks a wave (pick_ks; K <= 1024)
        (void)kb;
        if constexpr (EPI == GRX_GEMM_STORE)
            if (ns == 1) return go(I1{}, K4{});
        return go(I2{}, K4{});
    } else {
        if constexpr (EPI == GRX_GEMM_STORE) {
            if (ns == 1) {
                if (kb == 4) return go(I1{}, K4{});
                if (kb == 8) return go(I1{}, K8{});
                return go(I1{}, K16{});
            }
        }
        if (kb == 4) return go(I2{}, K4{});
        return go(I2{}, K8{});
    }
}

template <int EPI>
void launch_ks_fused(hipStream_t st, const grx_weight *w, const int8_t *xq, const float *xs, int m, const float *bias,
                     const GemmOut &o, int ns, int kb) {
    if (o.x == nullptr) return launch_ks_fused_pro<EPI, 0>(st, w, xq, xs, m, bias, o, ns, kb);
    if (o.ln_w2 == nullptr) return launch_ks_fused_pro<EPI, 1>(st, w, xq, xs, m, bias, o, ns, kb);
    return launch_ks_fused_pro<EPI, 2>(st, w, xq, xs, m, bias, o, ns, kb);
}

// Which kernel a product takes (GEMM_KERNEL forces one; tests force each
// with it): the one-row GEMV for one row (a conformer's one-row streaming
// chunk step, a single latent: the same blocks folded in the same order,
// its weights streamed once, on slices of the weight tiles where those
// give more workgroups: 1024 x 4096 6.2 us on 128 workgroups of 8 rows
// against 8.0 K-split; a forced GEMM_KERNEL keeps the matrix cores); the
// LDS-staged tiles from 256 rows on;
// below that the K-split tiles with their activations staged through LDS
// (at 224 rows: 1024 x 4096 17 us against 26 on the whole-K register walk
// and 50 on the LDS tiles, 4096 x 1024 12 against 19 and 15); without the
// staging, the K-split tiles up to 128 rows where the register walk has few
// tiles or a long K (at 126 rows: 4096 x 1024 10.4 us on the register walk
// against 11.9 K-split; 2048 x 1024 8.1 against 7.3; 1024 x 4096 25 against
// 19), the register walk otherwise.  The K-split kernel stages the
// activations through LDS unless told not to or they are not in 16-byte
// aligned whole groups of four blocks (a fused prologue builds them there).
enum Route { kRouteGemv1, kRouteLds, kRouteKs, kRouteMfma };
struct RoutePick {
    Route r;
    int ns, kb, da4;
    bool sa;
};
RoutePick pick_route(const grx_weight *w, const int8_t *xq, const float *xs, int m, const GemmOut &o) {
    const int kind = grx_tune(GRX_TUNE_GEMM_KERNEL);
    const bool pro = o.x != nullptr;
    RoutePick p{kRouteMfma, 1, 4, 0, false};
    if (m == 1 && kind < 0 && o.carry == nullptr && o.epi != GRX_GEMM_SCALE && w->nb > 0 &&
        grx_tune(GRX_TUNE_GEMV1) != 0) {
        p.r = kRouteGemv1;
        return p;
    }
    p.da4 = pro || (w->nb % 4 == 0 && ((uintptr_t)xs & 15) == 0) ? 1 : 0;
    p.sa = grx_tune(GRX_TUNE_GEMM_STAGE_A) != 0 && p.da4 && (pro || ((uintptr_t)xq & 15) == 0);
    const bool ks_ok = pick_ks(m, w->nb, w->rows, o.epi, o.carry != nullptr, p.sa, pro, &p.ns, &p.kb) &&
                       (kind == 2 || (p.sa ? m < 256 : (m <= 128 && (m <= 32 || w->rows <= 2048 || w->nb > 64))));
    if (kind == 3 || (kind != 1 && kind != 2 && m >= 256)) {
        p.r = kRouteLds;
    } else if (kind != 1 && ks_ok) {
        p.r = kRouteKs;
    } else {
        p.r = kRouteMfma;
    }
    return p;
}

bool fused_parts(const GemmOut &o) { return o.x != nullptr || o.epi == GRX_GEMM_GLU || o.ring.p != nullptr; }

}  // namespace

bool grx_gemm_q8_fuses(const grx_weight *w, int m, const GemmOut &o) {
    if (m <= 0 || w->rows == 0) return false;
    if (o.epi == GRX_GEMM_GLU && (w->rows % GRX_QK != 0 || o.lens == nullptr)) return false;
    if (o.ring.p != nullptr && o.epi != GRX_GEMM_STORE && o.epi != GRX_GEMM_GLU) return false;
    if (o.x != nullptr && (w->cols % GRX_QK != 0 || o.ln_w == nullptr || o.ln_b == nullptr)) return false;
    if (o.ln_w2 != nullptr && (o.x_out == nullptr || o.x_out == o.x || o.ln_b2 == nullptr)) return false;
    const RoutePick p = pick_route(w, nullptr, nullptr, m, o);
    if (p.r == kRouteGemv1)  // the one-row GEMV's prologue holds rows of up to 1280 values
        return (o.epi == GRX_GEMM_STORE || o.epi == GRX_GEMM_SILU_Q || o.epi == GRX_GEMM_GLU) &&
               (o.x == nullptr || w->nb * GRX_QK <= 1280);
    if (p.r == kRouteLds)  // the LDS tiles: GLU and ring copies, no prologue
        return o.x == nullptr;
    if (p.r != kRouteKs || !p.sa) return false;
    if (w->nb > ks_max_waves(p.ns, p.kb) * p.kb) return false;  // one run of blocks
    if (o.x != nullptr && (w->nb * GRX_QK > kKsProPieces * 256 || p.kb == 16 ||
                           grx_ceil_div(w->nb, p.kb) > kKsProWaves))
        return false;
    return true;
}

grx_status grx_gemm_q8_launch_ex(hipStream_t st, const grx_weight *w, const int8_t *xq, const float *xs, int m,
                                 const float *bias, const GemmOut &o) {
    if (m <= 0 || w->rows == 0) return GRX_OK;
    if (o.epi < GRX_GEMM_STORE || o.epi > GRX_GEMM_GLU)
        return grx_fail(GRX_EINVAL, "unknown product epilogue %d", o.epi);
    if ((o.epi == GRX_GEMM_SILU_Q || o.epi == GRX_GEMM_GLU) && w->rows % GRX_QK != 0)
        return grx_fail(GRX_ESIZE, "rounded or paired product output needs rows %% 32 == 0 (rows %d)", w->rows);
    const bool fused = fused_parts(o);
    if (fused && !grx_gemm_q8_fuses(w, m, o))
        return grx_fail(GRX_EINVAL, "a fused prologue, GLU or ring copy is not taken for %d rows of %dx%d", m,
                        w->rows, w->cols);
    const RoutePick p = pick_route(w, xq, xs, m, o);
    if (p.r == kRouteGemv1) {
        GemvArgs a = {};
        a.qs = w->qs;
        a.ds = w->ds;
        a.rows = w->rows;
        a.nb = w->nb;
        a.xq = xq;
        a.xs = xs;
        a.x = o.x;
        a.lda = o.lda;
        a.ln_w = o.ln_w;
        a.ln_b = o.ln_b;
        a.ln_w2 = o.ln_w2;
        a.ln_b2 = o.ln_b2;
        a.x_out = o.x_out;
        a.bias = bias;
        a.y = o.y;
        a.ldc = o.ldc;
        a.resid = o.y;
        a.ldr = o.ldc;
        a.yq = o.yq;
        a.ys = o.ys;
        a.ring = o.ring;
        a.lens = o.lens;
        a.T = o.T > 0 ? o.T : 1;
        a.cacheable = 0;  // weights streamed once a step
        const int epi = o.epi == GRX_GEMM_STORE ? GRX_EPI_STORE
                        : o.epi == GRX_GEMM_ADD ? GRX_EPI_RESID
                        : o.epi == GRX_GEMM_AXPY_HALF ? GRX_EPI_AXPY_HALF
                        : o.epi == GRX_GEMM_GLU ? GRX_EPI_GLU
                                                      : GRX_EPI_SILU_Q;
        const int pro = o.x == nullptr ? GRX_PRO_PREQ : o.ln_w2 != nullptr ? GRX_PRO_LN2 : GRX_PRO_LN;
        return grx_gemv_launch(st, 1, pro, epi, a, 0);
    }
    if (p.r == kRouteLds) {  // many rows: the LDS-staged 64 x 128 tiles
        dim3 g2(grx_ceil_div(m, 64), grx_ceil_div(w->tiles, 2));
#define GRX_GEMM_LDS(E)                                                                                           \
    case E:                                                                                                       \
        gemm_q8_lds_kernel<E><<<g2, kLdsThreads, 0, st>>>(w->qs, w->ds, w->rows, w->nb, w->tiles, xq, xs, m, bias, \
                                                          o.y, o.ldc, o.scale, o.yq, o.ys, ks_fuse(o));           \
        break;
        switch (o.epi) {
            GRX_GEMM_LDS(GRX_GEMM_STORE)
            GRX_GEMM_LDS(GRX_GEMM_ADD)
            GRX_GEMM_LDS(GRX_GEMM_AXPY_HALF)
            GRX_GEMM_LDS(GRX_GEMM_SCALE)
            GRX_GEMM_LDS(GRX_GEMM_SILU_Q)
            GRX_GEMM_LDS(GRX_GEMM_GLU)
        }
#undef GRX_GEMM_LDS
        GRX_LAUNCHED("gemm_q8_lds_kernel");
        return GRX_OK;
    }
    if (p.r == kRouteKs) {  // fewer rows: the K-split tiles
        if (fused) {
            switch (o.epi) {
                case GRX_GEMM_STORE: launch_ks_fused<GRX_GEMM_STORE>(st, w, xq, xs, m, bias, o, p.ns, p.kb); break;
                case GRX_GEMM_SILU_Q: launch_ks_fused<GRX_GEMM_SILU_Q>(st, w, xq, xs, m, bias, o, 2, p.kb); break;
                case GRX_GEMM_GLU: launch_ks_fused<GRX_GEMM_GLU>(st, w, xq, xs, m, bias, o, 2, p.kb); break;
                default: return grx_fail(GRX_EINVAL, "product epilogue %d takes no fused prologue", o.epi);
            }
            GRX_LAUNCHED("gemm_q8_kss_kernel");
            return GRX_OK;
        }
        switch (o.epi) {
            case GRX_GEMM_STORE:
                launch_ks_epi<GRX_GEMM_STORE>(st, w, xq, xs, m, bias, o, p.ns, p.kb, p.da4, p.sa);
                break;
            case GRX_GEMM_ADD: launch_ks_epi<GRX_GEMM_ADD>(st, w, xq, xs, m, bias, o, p.ns, p.kb, p.da4, p.sa); break;
            case GRX_GEMM_AXPY_HALF:
                launch_ks_epi<GRX_GEMM_AXPY_HALF>(st, w, xq, xs, m, bias, o, p.ns, p.kb, p.da4, p.sa);
                break;
            case GRX_GEMM_SCALE:
                launch_ks_epi<GRX_GEMM_SCALE>(st, w, xq, xs, m, bias, o, p.ns, p.kb, p.da4, p.sa);
                break;
            case GRX_GEMM_SILU_Q:
                launch_ks_epi<GRX_GEMM_SILU_Q>(st, w, xq, xs, m, bias, o, 2, p.kb, p.da4, p.sa);
                break;
        }
        GRX_LAUNCHED("gemm_q8_ks_kernel");
        return GRX_OK;
    }
    const int ns = pick_ns(m, w->rows, o.epi);
    dim3 grid(grx_ceil_div(m, 64), w->tiles * (4 / ns));
#define GRX_GEMM_GO(E, NS, U)                                                                                    \
    gemm_q8_mfma_kernel<E, NS, U><<<grid, 256, 0, st>>>(w->qs, w->ds, w->rows, w->nb, xq, xs, m, bias, o.y, o.ldc, \
                                                        o.scale, o.yq, o.ys)
#define GRX_GEMM_CASE(E)                \
    case E:                             \
        if (ns == 4)                    \
            GRX_GEMM_GO(E, 4, GRX_GEMM_U4); \
        else if (ns == 2)               \
            GRX_GEMM_GO(E, 2, GRX_GEMM_U2); \
        else                            \
            GRX_GEMM_GO(E, 1, GRX_GEMM_U1); \
        break;
    switch (o.epi) {
        GRX_GEMM_CASE(GRX_GEMM_STORE)
        GRX_GEMM_CASE(GRX_GEMM_ADD)
        GRX_GEMM_CASE(GRX_GEMM_AXPY_HALF)
        GRX_GEMM_CASE(GRX_GEMM_SCALE)
        case GRX_GEMM_SILU_Q:
            if (ns == 4)
                GRX_GEMM_GO(GRX_GEMM_SILU_Q, 4, GRX_GEMM_U4);
            else
                GRX_GEMM_GO(GRX_GEMM_SILU_Q, 2, GRX_GEMM_U2);
            break;
    }
#undef GRX_GEMM_CASE
#undef GRX_GEMM_GO
    GRX_LAUNCHED("gemm_q8_mfma_kernel");
    return GRX_OK;
}

// m rows of pre-rounded activations (xq [m][K], xs [m][K/32]) times the
// weight, into y (rows ldc apart), plus bias.
grx_status grx_gemm_q8_launch(hipStream_t st, const grx_weight *w, const int8_t *xq, const float *xs, int m,
                              const float *bias, float *y, int ldc) {
    GemmOut o;
    o.y = y;
    o.ldc = ldc;
    return grx_gemm_q8_launch_ex(st, w, xq, xs, m, bias, o);
}
