// q8_gemv_impl.h - device helpers shared by the one- and several-row
// Q8_0 products (q8_gemv.hip, q8_gemv1n.hip): weight loads, the int8 block
// dot, the activation row built and rounded by one wave (the products'
// prologues) and the products' epilogues.  Each translation unit gets its
// own copy (anonymous namespace).
#pragma once

#include <stdlib.h>

#include <type_traits>

#include "grx_internal.h"
#include "grx_ln.h"

namespace {

#ifndef GRX_GEMV_BU
#define GRX_GEMV_BU 8
#endif
#ifndef GRX_GEMV_NT
#define GRX_GEMV_NT 1
#endif
constexpr int BU = GRX_GEMV_BU;  // blocks whose loads are issued before any is used
// Several activation rows over several waves: the blocks go in rounds of
// kRound, each round's partial products through LDS, and wave m folds row
// m after every round (so LDS holds one round, not every block).
constexpr int kRound = 16;
// Pre-rounded activations of several rows (at most this many bytes: the
// host splits larger products into fewer rows) are copied to LDS;
// multi-row products may take up to kMultiLds bytes of LDS.
constexpr size_t kStageMax = 65536;
constexpr size_t kMultiLds = 128 * 1024;

// Weight loads are non-temporal: each weight byte is read once per product,
// and streaming it past the caches measured 6.7-6.8 TB/s on a 570 MB ring
// against 5.7-5.9 TB/s for ordinary loads (MI355X).
typedef int grx_v4i __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int4 wload(const int4 *p) {
#if GRX_GEMV_NT
    const grx_v4i v = __builtin_nontemporal_load(reinterpret_cast<const grx_v4i *>(p));
    return make_int4(v.x, v.y, v.z, v.w);
#else
    return *p;
#endif
}
__device__ __forceinline__ uint16_t wload(const uint16_t *p) {
#if GRX_GEMV_NT
    return __builtin_nontemporal_load(p);
#else
    return *p;
#endif
}

// ---------------------------------------------------------------- helpers

__device__ __forceinline__ int sdot8(const int4 &w0, const int4 &w1, const int4 &a0, const int4 &a1) {
    int s = 0;
    s = __builtin_amdgcn_sdot4(w0.x, a0.x, s, false);
    s = __builtin_amdgcn_sdot4(w0.y, a0.y, s, false);
    s = __builtin_amdgcn_sdot4(w0.z, a0.z, s, false);
    s = __builtin_amdgcn_sdot4(w0.w, a0.w, s, false);
    s = __builtin_amdgcn_sdot4(w1.x, a1.x, s, false);
    s = __builtin_amdgcn_sdot4(w1.y, a1.y, s, false);
    s = __builtin_amdgcn_sdot4(w1.z, a1.z, s, false);
    s = __builtin_amdgcn_sdot4(w1.w, a1.w, s, false);
    return s;
}

// Round (M rows x nb blocks) of float32 activations in LDS or global memory
// into LDS, 32 lanes per block: lane e holds value e, the block's largest
// magnitude comes from five xor-shuffles within the 32 lanes (the maximum
// is order-free), and each lane rounds its own value as grx_quant_block does.
template <int M>
__device__ __forceinline__ void quant_into_lds(const float *src, int ld, int nb, int8_t *lxq,
                                               float *lxs, int tid, int nthreads) {
    const int K = nb * GRX_QK;
    const int e = tid & 31;
    for (int g = tid >> 5; g < M * nb; g += nthreads >> 5) {
        const int m = g / nb, b = g - m * nb;
        const float v = src[(size_t)m * ld + b * GRX_QK + e];
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
        lxq[(size_t)m * K + b * GRX_QK + e] = (int8_t)(int)r;
        if (e == 0) lxs[m * nb + b] = __fmul_rn(amax, grx_bits_f32(0x3c010204u));
    }
}

// ---------------------------------------------------------------- one row

// The largest of each 8 lanes' values (a Q8_0 block held as 8 float4s).
__device__ __forceinline__ float max8(float m) {
    float t = dpp_f32<kDppXor1>(m);
    m = t > m ? t : m;
    t = dpp_f32<kDppXor2>(m);
    m = t > m ? t : m;
    t = dpp_f32<kDppHalfMirror>(m);
    return t > m ? t : m;
}
__device__ __forceinline__ float amax4(const float4 &v) {
    float m = fabsf(v.x);
    m = m > 0.0f ? m : 0.0f;
    float t = fabsf(v.y);
    m = t > m ? t : m;
    t = fabsf(v.z);
    m = t > m ? t : m;
    t = fabsf(v.w);
    return t > m ? t : m;
}
__device__ __forceinline__ uint32_t quant4(const float4 &v, float id) {
    auto q = [&](float x) {
        float r = rintf(__fmul_rn(x, id));
        r = fminf(fmaxf(r, -128.0f), 127.0f);
        return (uint32_t)(uint8_t)(int8_t)(int)r;
    };
    return q(v.x) | q(v.y) << 8 | q(v.z) << 16 | q(v.w) << 24;
}

// Widest row a one-row product rounds in its prologue: NP pieces of 4
// values per lane held in registers (NP = 2, 4 or 5: up to 512, 1024 or
// 1280 values).
constexpr int kRowPieces = 5;
// Blocks whose weight loads a one-row product issues before its prologue.
constexpr int kPrefetch = 4;
// Row stride (floats) of the key rows staged for XSCORES: 16-byte reads of
// a row per lane land in distinct banks.
constexpr int kKeyLd = 68;

// Activation row m of a product, built by ONE wave (every lane active) and
// rounded to Q8_0 into LDS (lxq [.][K], lxs [.][nb]): the row as NP float4
// pieces per lane (piece P = 64 j + lane, K <= 256 NP), then by PRO
//   QUANT     quantU8 of x row m (q8int.go:88-105)
//   LN        layerNorm (internal/kern/mathx.go:55-75), then quantU8
//   EMBED_LN  the whisper embedding row (tok[m] at the position), stored to
//             x_out row m by tile 0, then as LN
//   LN64      layerNorm of pockettts/nn.go:27-49, then quantU8
// with cross-lane DPP sums (float64) and maxima: no workgroup barrier.
// after_loads() runs once the row's loads are issued (the caller's own
// loads go there).
template <int NP, int PRO, typename After>
__device__ __forceinline__ void wave_row_prologue(const GemvArgs &a, int m, int8_t *lxq, float *lxs, int lane,
                                                  int tile, After after_loads, int ldq = 0) {
    const int nb = a.nb, K = nb * GRX_QK;
    const size_t rq = ldq > 0 ? (size_t)ldq : (size_t)K;  // bytes between the rounded rows in lxq
    const int npc = K / 4;  // float4 pieces
    constexpr bool L2 = PRO == GRX_PRO_LN2;
    float4 xv[NP], wv[NP], bv[NP], wv2[L2 ? NP : 1], bv2[L2 ? NP : 1];
    const float4 *x4 = reinterpret_cast<const float4 *>(a.x + (size_t)m * a.lda);
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        const int P = min(j * 64 + lane, npc - 1);
        if constexpr (PRO == GRX_PRO_EMBED_LN) {
            // tokEmb.row(tok) + decPos[pos] (whisper/decoder.go:42-46):
            // the embedding row from its tile layout, d*q then + pos
            const int t = a.tok[m], p = *a.pos + a.pos_add + (a.streams ? 0 : m);
            const int etile = t >> 6, elane = t & 63, i = 4 * P;
            const int b = i >> 5, h = (i >> 4) & 1, e = i & 15;
            const uint32_t q4 = *reinterpret_cast<const uint32_t *>(
                a.emb_qs + (((size_t)etile * nb + b) * 2 + h) * 1024 + elane * 16 + e);
            const float d = grx_f16_to_f32(a.emb_ds[((size_t)etile * nb + b) * 64 + elane]);
            const float4 pe = reinterpret_cast<const float4 *>(a.pos_emb + (size_t)p * K)[P];
            xv[j].x = __fadd_rn(__fmul_rn((float)(int8_t)(q4 & 0xff), d), pe.x);
            xv[j].y = __fadd_rn(__fmul_rn((float)(int8_t)((q4 >> 8) & 0xff), d), pe.y);
            xv[j].z = __fadd_rn(__fmul_rn((float)(int8_t)((q4 >> 16) & 0xff), d), pe.z);
            xv[j].w = __fadd_rn(__fmul_rn((float)(int8_t)(q4 >> 24), d), pe.w);
        } else {
            xv[j] = x4[P];
        }
        if constexpr (PRO == GRX_PRO_LN || PRO == GRX_PRO_EMBED_LN || PRO == GRX_PRO_LN64 || L2) {
            if (PRO != GRX_PRO_LN64 || a.ln_w != nullptr) {
                wv[j] = reinterpret_cast<const float4 *>(a.ln_w)[P];
                bv[j] = reinterpret_cast<const float4 *>(a.ln_b)[P];
            }
        }
        if constexpr (L2) {
            wv2[j] = reinterpret_cast<const float4 *>(a.ln_w2)[P];
            bv2[j] = reinterpret_cast<const float4 *>(a.ln_b2)[P];
        }
    }
    // loads issued behind this row's (they complete in order): waiting for
    // the row does not wait for them
    after_loads();
    if constexpr (PRO == GRX_PRO_EMBED_LN) {
        if (tile == 0) {
#pragma unroll
            for (int j = 0; j < NP; ++j)
                if (j * 64 + lane < npc) reinterpret_cast<float4 *>(a.x_out + (size_t)m * a.lda)[j * 64 + lane] = xv[j];
        }
    }
    if constexpr (PRO == GRX_PRO_LN || PRO == GRX_PRO_EMBED_LN || L2) {
        // layerNorm (internal/kern/mathx.go:55-75): float64 sums (in the
        // reference's order where the tree's could round differently),
        // mean and inv rounded to float32, y = (v-mean)*inv*w + b
        wave_ln32<NP>(xv, wv, bv, npc, lane);
        if constexpr (L2) {
            // a block's norm_out (conformer/encoder.go:426) kept by tile 0,
            // then the next block's first LayerNorm
            if (tile == 0) {
#pragma unroll
                for (int j = 0; j < NP; ++j)
                    if (j * 64 + lane < npc) reinterpret_cast<float4 *>(a.x_out + (size_t)m * a.lda)[j * 64 + lane] = xv[j];
            }
            wave_ln32<NP>(xv, wv2, bv2, npc, lane);
        }
    } else if constexpr (PRO == GRX_PRO_LN64) {
        // layerNorm of pockettts/nn.go:27-49: statistics and the
        // normalized value in float64, gain and bias in float32
        wave_ln64<NP>(xv, wv, bv, a.ln_w != nullptr, npc, lane, a.ln_eps, [&](float4 (&v)[NP]) {
#pragma unroll
            for (int j = 0; j < NP; ++j) v[j] = x4[min(j * 64 + lane, npc - 1)];
        });
    }
    // quantU8 (q8int.go:88-105): a block is 8 pieces in 8 lanes
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        const int P = j * 64 + lane;
        const float amax = max8(amax4(xv[j]));
        const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
        const uint32_t q = quant4(xv[j], id);
        if (P < npc) {
            reinterpret_cast<uint32_t *>(lxq + (size_t)m * rq)[P] = q;
            if ((lane & 7) == 0) lxs[m * nb + (P >> 3)] = __fmul_rn(amax, grx_bits_f32(0x3c010204u));
        }
    }
}

// The products' epilogues: row m of the tile's 64 outputs (acc[m] in lane
// `lane`) is ended by wave 0, or by wave m % W when rows were folded round
// by round (RND).
template <int M, int W, bool RND, int EPI>
__device__ __forceinline__ void gemv_epilogue(const GemvArgs &a, const float (&acc)[M], int row, int lane,
                                              int wave, int pos0) {
    auto mine = [&](int m) { return !RND || m % W == wave; };
    if constexpr (EPI == GRX_EPI_ARGMAX) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            if (!mine(m)) continue;
            const float c = acc[m];
            if (a.y != nullptr && row < a.rows) a.y[(size_t)m * a.ldc + row] = c;
            // key: orderable float bits, then the complement of the index, so
            // the maximum key is the largest value at its first index
            // (whisper/transcribe.go:459-464); -0 counts as +0 and NaN never wins.
            unsigned long long key = 0;
            if (row < a.rows && !(c != c)) {
                const float cc = c == 0.0f ? 0.0f : c;
                const uint32_t u = __float_as_uint(cc);
                const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
                key = ((unsigned long long)ord << 32) | (uint32_t)(0xffffffffu - (uint32_t)row);
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const unsigned long long k2 = __shfl_xor(key, o);
                key = k2 > key ? k2 : key;
            }
            if (lane == 0) {
                if (a.keys != nullptr) {
                    // one slot per workgroup and row: no contended atomics;
                    // argmax_finish_kernel takes the maximum afterwards
                    a.keys[(size_t)blockIdx.x * M + m] = key;
                } else {
                    // a returning atomic: its old value comes back only once
                    // the maximum has been taken at the coherence point
                    const unsigned long long old = atomicMax(a.amax + m, key);
                    asm volatile("; argmax done %0" ::"v"((uint32_t)old));
                }
            }
        }
        if (a.counter != nullptr) {
            // The last workgroup to finish ends the decode step: the argmax
            // token, its record, the next position; then clears the key and
            // the counter for the next step.  Device-scope atomics are
            // coherent across the XCDs, and each workgroup's atomicMax has
            // returned before its count is added, so no cache writeback is
            // needed.  (Rows folded by several waves: every wave's atomicMax
            // is in before wave 0 counts.)
            if constexpr (RND) __syncthreads();
            if (wave != 0) return;
            unsigned int done = 0;
            if (lane == 0) done = atomicAdd(a.counter, 1u);
            done = __shfl(done, 0);
            if (done == gridDim.x - 1) {
                const int p0 = *a.pos;
                if (lane < M) {
                    const unsigned long long k = atomicMax(a.amax + lane, 0ull);
                    const int t = (int)(0xffffffffu - (uint32_t)(k & 0xffffffffull));
                    a.tok_w[lane] = t;
                    if (a.streams)
                        a.hist[(size_t)lane * a.hist_stream + p0] = t;
                    else
                        a.hist[p0 + lane] = t;
                    a.amax[lane] = 0ull;
                }
                if (lane == 0) {
                    *a.pos_w = p0 + (a.streams ? 1 : M);
                    *a.counter = 0u;
                }
            }
        }
        return;
    }
    if constexpr (EPI == GRX_EPI_GLU) {
        // rows paired (grx_glu_row): lane l < 16 of each 32-row half holds
        // channel 16*(row/32) + l's a-row, lane l + 16 its b-row
#pragma unroll
        for (int m = 0; m < M; ++m) {
            if (!mine(m)) continue;
            const float b = __shfl_xor(acc[m], 16);
            if (row >= a.rows || (lane & 16) != 0) continue;
            const int ch = (row >> 5) * 16 + (lane & 15);
            const int s = m / a.T;
            const float v = m - s * a.T < a.lens[s] ? grx_glu_pair(acc[m], b) : 0.0f;
            a.y[(size_t)m * a.ldc + ch] = v;
            if (a.ring.p != nullptr) ring_put(a.ring, ring_row(a.ring, ring_head(a.ring), m), ch - a.ring.col0, v);
        }
        return;
    }
    if constexpr (EPI == GRX_EPI_AXPY_HALF) {
        // the matrix-core product's AXPY_HALF: y = fma(0.5, c, resid)
#pragma unroll
        for (int m = 0; m < M; ++m) {
            if (!mine(m)) continue;
            if (row < a.rows) a.y[(size_t)m * a.ldc + row] = __fmaf_rn(0.5f, acc[m], a.resid[(size_t)m * a.ldr + row]);
        }
        return;
    }
    if constexpr (EPI == GRX_EPI_SILU_Q) {
        // the matrix-core product's SILU_Q: v = c / (EXP8(-c) + 1), then
        // quantU8 of its 32-value blocks (rows 64*tile..+31 and +32..+63,
        // rows % 32 == 0) into yq [M][rows], ys [M][rows/32]
#pragma unroll
        for (int m = 0; m < M; ++m) {
            if (!mine(m)) continue;
            const float x = acc[m];
            const float v = row < a.rows ? __fdiv_rn(x, __fadd_rn(grx_exp8(__fsub_rn(0.0f, x)), 1.0f)) : 0.0f;
            const float av = fabsf(v);
            float amax = av > 0.0f ? av : 0.0f;
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) {
                const float t = __shfl_xor(amax, o, 32);
                amax = t > amax ? t : amax;
            }
            if (row < a.rows) {
                const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
                float r = rintf(__fmul_rn(v, id));
                r = fminf(fmaxf(r, -128.0f), 127.0f);
                a.yq[(size_t)m * a.rows + row] = (int8_t)(int)r;
                if ((lane & 31) == 0) a.ys[(size_t)m * (a.rows >> 5) + (row >> 5)] = __fmul_rn(amax, grx_bits_f32(0x3c010204u));
            }
        }
        return;
    }
    if constexpr (EPI == GRX_EPI_GELU_Q) {
        // geluVec, then quantU8 of the output's 32-value blocks for the next
        // product: rows 64*tile..+31 and +32..+63 are two whole blocks
        // (rows % 32 == 0), held by the two halves of this wave.
#pragma unroll
        for (int m = 0; m < M; ++m) {
            if (!mine(m)) continue;
            // streams: each row is its own [1][rows] buffer
            const int flat = a.streams ? row : m * a.rows + row, total = a.streams ? a.rows : M * a.rows;
            const int start = flat & ~((1 << 14) - 1);
            const int len = min(1 << 14, total - start);
            const float v = row < a.rows ? grx_gelu_at(acc[m], flat - start, len) : 0.0f;
            const float av = fabsf(v);
            float amax = av > 0.0f ? av : 0.0f;
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) {
                const float t = __shfl_xor(amax, o, 32);
                amax = t > amax ? t : amax;
            }
            if (row < a.rows) {
                const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
                float r = rintf(__fmul_rn(v, id));
                r = fminf(fmaxf(r, -128.0f), 127.0f);
                a.y[(size_t)m * a.ldc + row] = v;
                a.yq[(size_t)m * a.rows + row] = (int8_t)(int)r;
                if ((lane & 31) == 0) a.ys[(size_t)m * (a.rows >> 5) + (row >> 5)] = __fmul_rn(amax, grx_bits_f32(0x3c010204u));
            }
        }
        return;
    }
    if constexpr (EPI == GRX_EPI_QKV_ROPE) {
        // applyRope (pockettts/nn.go:80-93) on the q and k rows: the pair
        // (2i, 2i+1) of a head sits in adjacent lanes; x'[2i] = r*c - im*s,
        // x'[2i+1] = r*s + im*c, unfused, with f32 cos/sin of the angle.
#pragma unroll
        for (int m = 0; m < M; ++m) {
            if (!mine(m)) continue;
            const float c = acc[m];
            const float other = __shfl_xor(c, 1);
            if (row >= a.rows) continue;
            const int pos = pos0 + a.pos_add + m;
            if (row < 2 * a.seg) {
                const int j = row % a.seg, hd = 2 * a.rope_half;
                const int i = (j % hd) >> 1;
                const float cs = a.rope_cos[(size_t)pos * a.rope_half + i];
                const float sn = a.rope_sin[(size_t)pos * a.rope_half + i];
                const bool even = (j & 1) == 0;
                const float r = even ? c : other, im = even ? other : c;
                const float v = even ? __fsub_rn(__fmul_rn(r, cs), __fmul_rn(im, sn))
                                     : __fadd_rn(__fmul_rn(r, sn), __fmul_rn(im, cs));
                if (row < a.seg)
                    a.y[(size_t)m * a.ldc + row] = v;
                else
                    a.kc[(size_t)pos * a.seg + row - a.seg] = v;
            } else {
                a.vc[(size_t)pos * a.seg + row - 2 * a.seg] = c;
            }
        }
        return;
    }
    if (row >= a.rows) return;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        if (!mine(m)) continue;
        const float c = acc[m];
        if constexpr (EPI == GRX_EPI_STORE) {
            a.y[(size_t)m * a.ldc + row] = c;
        } else if constexpr (EPI == GRX_EPI_RESID) {
            a.y[(size_t)m * a.ldc + row] = __fadd_rn(a.resid[(size_t)m * a.ldr + row], c);
        } else if constexpr (EPI == GRX_EPI_GELU) {
            // parGelu (whisper/encoder.go:147-151): geluVec over chunks of
            // 1<<14 values of the flat [M][rows] output.
            const int flat = a.streams ? row : m * a.rows + row, total = a.streams ? a.rows : M * a.rows;
            const int start = flat & ~((1 << 14) - 1);
            const int len = min(1 << 14, total - start);
            a.y[(size_t)m * a.ldc + row] = grx_gelu_at(c, flat - start, len);
        } else if constexpr (EPI == GRX_EPI_QKV) {
            // one stream: rows are positions pos.., caches [pos][seg];
            // streams: row m at pos in stream m's cache (kv_stream floats on)
            const int pos = pos0 + a.pos_add + (a.streams ? 0 : m);
            const size_t so = a.streams ? (size_t)m * a.kv_stream : 0;
            if (row < a.seg)
                a.y[(size_t)m * a.ldc + row] = c;
            else if (row < 2 * a.seg)
                a.kc[so + (size_t)pos * a.seg + row - a.seg] = c;
            else
                a.vc[so + (size_t)pos * a.seg + row - 2 * a.seg] = c;
        }
    }
}


}  // namespace
// q8_gemv1n.hip: one-row products on slices of `rows` (8, 16 or 32) rows of
// the 64-row tiles; grx_gemv1_rows picks the slice (64: whole tiles, the
// one-row kernel of q8_gemv.hip) for a product of `tiles` tiles.
int grx_gemv1_rows(int tiles, int pro, int epi);
hipError_t grx_gemv1n_launch(hipStream_t st, const GemvArgs &a, int tiles, int rows, int pro, int epi);
