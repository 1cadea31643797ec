// whisper_sample.hip - whisper's token rules and sampler on the device.
//
// session.process and session.sample (whisper/transcribe.go:370-494 of
// github.com/xattribution/gorelaxor) over one row of logits, in one
// workgroup of 1024 threads, thread t holding entries [t*CH, t*CH+CH) in
// registers:
//   temperature division, the suppression rules (special tokens, languages,
//   the suppress list, timestamp pairs, the initial timestamp limit, no
//   timestamp before the last one), logSoftmax, the rule that timestamps
//   together outweighing every text token force a timestamp, softmaxInf,
//   then the argmax (temperature 0) or the draw of a cumulative sum against
//   the caller's uniform r, and the best timestamp.
//
// The reference's sums (logSoftmax's, the timestamps' and the draw's) are
// float32 sums left to right over ~52k entries; their results are kept bit
// for bit by keeping that order.  A term smaller than half an ulp of the
// running sum cannot change it (round to nearest), and the running sum of
// non-negative terms is never below the largest earlier term M, so a term
// below ulp(M)/2 is skipped; the terms that remain are written to LDS in
// index order (several rounds when they do not fit) and one lane adds them.
// With real logits few terms remain; in the worst case all do.
#include <math.h>

#include "grx_float.h"
#include "grx_internal.h"

namespace {

constexpr int kThreads = 1024;
constexpr int kRing = 16384;  // LDS slots for the remaining terms of one round
constexpr int kMaxLogits = kThreads * 64;

// a float's ulp/2: the smallest term that can change a sum of at least m
// (0 when m is zero or subnormal, where every nonzero term counts)
__device__ __forceinline__ float half_ulp(float m) {
    const unsigned e = (__float_as_uint(m) >> 23) & 0xff;
    return e <= 24 ? 0.f : __uint_as_float((e - 24) << 23);
}

// block-wide exclusive scans over kThreads values (sum of ints, max of
// floats); `red` holds kThreads/64 slots
__device__ int block_excl_sum(int v, int *red, int *total) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    int x = v;
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    if (lane == 63) red[w] = x;
    __syncthreads();
    int base = 0, all = 0;
    for (int i = 0; i < kThreads / 64; ++i) {
        base += i < w ? red[i] : 0;
        all += red[i];
    }
    __syncthreads();
    *total = all;
    return base + x - v;
}

__device__ float block_excl_max(float v, float *red) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    float x = v;
    for (int o = 1; o < 64; o <<= 1) {
        const float y = __shfl_up(x, o);
        if (lane >= o) x = fmaxf(x, y);
    }
    float ex = __shfl_up(x, 1);
    if (lane == 0) ex = 0.f;
    if (lane == 63) red[w] = x;
    __syncthreads();
    float base = 0.f;
    for (int i = 0; i < w; ++i) base = fmaxf(base, red[i]);
    __syncthreads();
    return fmaxf(base, ex);
}

__device__ float block_max(float v, float *red) {
    const int t = threadIdx.x;
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    if ((t & 63) == 0) red[t >> 6] = v;
    __syncthreads();
    float m = red[0];
    for (int i = 1; i < kThreads / 64; ++i) m = fmaxf(m, red[i]);
    __syncthreads();
    return m;
}

// the first index of the largest value (ties to the lower index)
__device__ void block_argmax(float v, int i, float *redv, int *redi, float *best_v, int *best_i) {
    const int t = threadIdx.x;
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o);
        const int oi = __shfl_xor(i, o);
        const bool take = ov > v || (ov == v && oi < i);
        v = take ? ov : v;
        i = take ? oi : i;
    }
    if ((t & 63) == 0) {
        redv[t >> 6] = v;
        redi[t >> 6] = i;
    }
    __syncthreads();
    float bv = redv[0];
    int bi = redi[0];
    for (int k = 1; k < kThreads / 64; ++k)
        if (redv[k] > bv || (redv[k] == bv && redi[k] < bi)) {
            bv = redv[k];
            bi = redi[k];
        }
    __syncthreads();
    *best_v = bv;
    *best_i = bi;
}

struct SampleShared {
    __align__(16) float ring[kRing];
    int ring_i[kRing];
    unsigned mask[65536 / 32];
    float redf[kThreads / 64];
    int redi[kThreads / 64];
    float bcast_f[4];
    int bcast_i[4];
};

// Left-to-right float32 sum over the block (index order), from 0, of
// term(j) for each thread's entries j < CH (CH <= 64); the terms that cannot
// change the sum are skipped.  draw: stop at the first index where r < sum
// (returned in *hit, -1 if none).  term() is called up to three times per
// entry.
template <int CH, typename Term>
__device__ float seq_sum(Term term, SampleShared &sh, bool draw, float r, int *hit, int *terms) {
    const int t = threadIdx.x;
    float lmax = 0.f;
    unsigned long long keep = 0;  // bit j: term j may change the sum
    #pragma unroll 1
    for (int j0 = 0; j0 < CH; j0 += 4) {
        float tv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) tv[u] = term(j0 + u);
#pragma unroll
        for (int u = 0; u < 4; ++u) lmax = fmaxf(lmax, tv[u]);
    }
    float m = block_excl_max(lmax, sh.redf);
    #pragma unroll 1
    for (int j0 = 0; j0 < CH; j0 += 4) {
        float tv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) tv[u] = term(j0 + u);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            keep |= (unsigned long long)(tv[u] > 0.f && tv[u] >= half_ulp(m)) << (j0 + u);
            m = fmaxf(m, tv[u]);
        }
    }
    int total;
    const int base = block_excl_sum(__popcll(keep), sh.redi, &total);
    float sum = 0.f;
    int found = -1;
    for (int r0 = 0; r0 < total; r0 += kRing) {
        // this round's terms into the ring, in index order
        if (base < r0 + kRing && base + __popcll(keep) > r0) {
            int rank = base;
#pragma unroll 1
            for (int j0 = 0; j0 < CH; j0 += 4) {
                const unsigned kb = (unsigned)(keep >> j0) & 0xfu;
                if (kb == 0u) continue;
                float tv[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) tv[u] = term(j0 + u);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if ((kb >> u) & 1u) {
                        if (rank >= r0 && rank < r0 + kRing) {
                            sh.ring[rank - r0] = tv[u];
                            sh.ring_i[rank - r0] = t * CH + j0 + u;
                        }
                        ++rank;
                    }
                }
            }
        }
        __syncthreads();
        if (t == 0) {
            const int n = min(kRing, total - r0);
            int k = 0;
            if (!draw) {
                // 64 terms per step: their 16 reads issued at once, each
                // add waiting only for the read that brings its term
                const float4 *q = reinterpret_cast<const float4 *>(sh.ring);
                const int nq = n / 64 * 16;  // float4s in whole steps
                for (int b = 0; b < nq; b += 16) {
                    float4 c[16];
#pragma unroll
                    for (int u = 0; u < 16; ++u) c[u] = q[b + u];
#pragma unroll
                    for (int u = 0; u < 16; ++u) {
                        sum = __fadd_rn(sum, c[u].x);
                        sum = __fadd_rn(sum, c[u].y);
                        sum = __fadd_rn(sum, c[u].z);
                        sum = __fadd_rn(sum, c[u].w);
                    }
                }
                for (k = nq * 4; k < n; ++k) sum = __fadd_rn(sum, sh.ring[k]);
            } else {
                for (; k < n; ++k) {
                    sum = __fadd_rn(sum, sh.ring[k]);
                    if (r < sum) {
                        found = sh.ring_i[k];
                        break;
                    }
                }
            }
            sh.bcast_f[0] = sum;
            sh.bcast_i[0] = found;
        }
        __syncthreads();
        sum = sh.bcast_f[0];
        found = sh.bcast_i[0];
        __syncthreads();
        if (found >= 0) break;
    }
    *hit = found;
    *terms = total;
    return sum;
}

// float32(log(float64(s))) + m, as the reference forms the log of a sum
__device__ __forceinline__ float log_plus(float s, float m) { return __fadd_rn((float)log((double)s), m); }

// One row of logits through the rules and the sampler.  Each thread owns
// entries [t*ch, t*ch + ch); its masked logits live in vg and its terms (then
// probabilities) in g, both [ch][1024] floats of device scratch (entry j of
// thread t at j*1024 + t, so a wave's accesses are contiguous) that only the
// owning thread reads and writes.  The logits themselves are read once,
// coalesced, through LDS.
// In loop form (la.st set) the sequence state comes from the device, the
// draw from la.rs, and the chosen token goes to the loop's record and the
// decoder's next token, the state moving on as transcribe.go:211-237 moves
// it; a sequence done or failed is left alone.
template <int CH>
__global__ __launch_bounds__(kThreads) void sample_kernel(const float *__restrict__ logits, GrxSampleArgs a,
                                                          const int *__restrict__ suppress, float *__restrict__ vg,
                                                          float *__restrict__ g, GrxSampleOut *__restrict__ out,
                                                          const GrxLoopArgs la) {
    static_assert(CH % 4 == 0, "entries per thread in groups of four");
    constexpr int ch = CH;
    extern __shared__ __align__(16) unsigned char smem[];
    SampleShared &sh = *reinterpret_cast<SampleShared *>(smem);
    const int t = threadIdx.x, n = a.n, i0 = t * ch;
    const float ninf = -INFINITY;
    GrxLoopDev lst{};
    if (la.st != nullptr) {
        lst = *la.st;  // the same for every thread: the return below is uniform
        if (lst.done || lst.failed || lst.i >= la.n_max) return;
        a.initial = lst.n_tokens == 0;
        a.last = lst.n_tokens > 0 && lst.last >= a.beg;
        a.penult = lst.n_tokens < 2 || lst.penult >= a.beg;
        a.has_ts = lst.has_ts;
        a.seek_delta = lst.seek_delta;
        if (la.rs != nullptr) a.r = la.rs[lst.i];
    }
    // the suppress list and the single special tokens into a bitmap
    for (int i = t; i < (n + 31) / 32; i += kThreads) sh.mask[i] = 0u;
    __syncthreads();
    auto mark = [&](int id) {
        if (id >= 0 && id < n) atomicOr(&sh.mask[id >> 5], 1u << (id & 31));
    };
    for (int i = t; i < a.n_suppress; i += kThreads) mark(suppress[i]);
    if (t == 0) {
        mark(a.not_);
        mark(a.sot);
        mark(a.nosp);
        mark(a.solm);
        mark(a.translate);
        mark(a.transcribe);
        mark(a.prev);
        if (a.initial) {
            mark(a.eot);
            mark(a.space);
        }
    }
    __syncthreads();
    // vt[j], gt[j]: entry j of this thread
    struct Col {
        float *p;
        __device__ float &operator[](int j) const { return p[(size_t)j * kThreads]; }
    };
    const Col vt{vg + t}, gt{g + t};
    // the logits, kRing at a time through LDS, each thread taking its own
    for (int r0 = 0; r0 < n; r0 += kRing) {
        const int m = min(kRing, n - r0);
        for (int k = t; k < m; k += kThreads) sh.ring[k] = logits[r0 + k];
        __syncthreads();
        const int lo = max(i0, r0), hi = min(i0 + ch, r0 + m);
        for (int i = lo; i < hi; ++i) vt[i - i0] = sh.ring[i - r0];
        __syncthreads();
    }
    // process() (transcribe.go:370-426): the temperature, then the rules.
    // Loops run in groups of four entries whose loads are issued together.
    float lm = ninf;
    #pragma unroll 1
    for (int j0 = 0; j0 < CH; j0 += 4) {
        float xv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) xv[u] = vt[j0 + u];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = i0 + j0 + u;
            float x = xv[u];
            if (a.temp > 0.f) x = __fdiv_rn(x, a.temp);
            const int ic = min(i, n - 1);
            bool off = i >= n || ((sh.mask[ic >> 5] >> (ic & 31)) & 1u);
            off |= i >= a.sot + 1 && i < a.sot + 1 + a.n_lang;
            off |= a.last && a.penult && i >= a.beg;
            off |= a.last && !a.penult && i < a.eot;
            off |= a.initial && i >= a.beg + a.tid0 + 1;
            off |= a.has_ts && i >= a.beg && i < a.beg + a.seek_delta / 2;
            x = off ? ninf : x;
            vt[j0 + u] = x;
            lm = fmaxf(lm, x);
        }
    }
    // logSoftmax (transcribe.go:495-514)
    const float mx = block_max(lm, sh.redf);
    auto exps = [&](float m) {  // the terms expf(v - m) into g (0 for -inf)
        #pragma unroll 1
        for (int j0 = 0; j0 < CH; j0 += 4) {
            float xv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) xv[u] = vt[j0 + u];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float e = grx_expf_go(__fsub_rn(xv[u], m));
                gt[j0 + u] = xv[u] > ninf ? e : 0.f;
            }
        }
    };
    exps(mx);
    auto from_g = [&](int j) { return gt[j]; };
    int hit, terms, unused;
    const float s = seq_sum<CH>(from_g, sh, false, 0.f, &hit, &terms);
    const float ls = log_plus(s, mx);
    // timestamps together against the best text token (transcribe.go:427-446)
    float tsm = ninf, txm = ninf;
    #pragma unroll 1
    for (int j0 = 0; j0 < CH; j0 += 4) {
        float xv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) xv[u] = vt[j0 + u];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float lp = xv[u] > ninf ? __fsub_rn(xv[u], ls) : ninf;
            const bool ts = i0 + j0 + u >= a.beg;
            tsm = ts ? fmaxf(tsm, lp) : tsm;
            txm = ts ? txm : fmaxf(txm, lp);
        }
    }
    const float tsMax = block_max(tsm, sh.redf);
    const float textMax = block_max(txm, sh.redf);
    bool force_ts = false;
    if (tsMax > ninf) {
        const bool mine = i0 + CH > a.beg;  // this thread holds timestamps
        auto ts_term = [&](int j) {
            float e = 0.f;
            if (mine) {
                const float x = vt[j];
                const float t2 = grx_expf_go(__fsub_rn(__fsub_rn(x, ls), tsMax));
                e = i0 + j >= a.beg && x > ninf ? t2 : 0.f;
            }
            return e;
        };
        const float tss = seq_sum<CH>(ts_term, sh, false, 0.f, &hit, &unused);
        force_ts = log_plus(tss, tsMax) > textMax;
    }
    // softmaxInf of the logits (transcribe.go:517-536): when no text token
    // was taken away, its maximum and sum are logSoftmax's
    float s2 = s;
    if (force_ts) {
        lm = ninf;
        #pragma unroll 1
        for (int j0 = 0; j0 < CH; j0 += 4) {
            float xv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) xv[u] = vt[j0 + u];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float x = i0 + j0 + u < a.beg ? ninf : xv[u];
                vt[j0 + u] = x;
                lm = fmaxf(lm, x);
            }
        }
        const float mx2 = block_max(lm, sh.redf);
        exps(mx2);
        s2 = seq_sum<CH>(from_g, sh, false, 0.f, &hit, &unused);
    }
    // the probabilities, in g; the first largest of all, and from beg
    float lv = -1.f, lt = -1.f;
    int li = 0, lti = a.beg;
    #pragma unroll 1
    for (int j0 = 0; j0 < CH; j0 += 4) {
        float ev[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) ev[u] = gt[j0 + u];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = i0 + j0 + u;
            const float p = __fdiv_rn(ev[u], s2);
            gt[j0 + u] = p;
            const bool b1 = p > lv, b2 = i >= a.beg && i < n && p > lt;
            lv = b1 ? p : lv;
            li = b1 ? i : li;
            lt = b2 ? p : lt;
            lti = b2 ? i : lti;
        }
    }
    // sample() (transcribe.go:449-494)
    float bv, tv;
    int id, tid;
    block_argmax(lv, li, sh.redf, sh.redi, &bv, &id);
    block_argmax(lt, lti, sh.redf, sh.redi, &tv, &tid);
    if (a.temp != 0.f) {
        int drawn;
        seq_sum<CH>(from_g, sh, true, a.r, &drawn, &unused);
        if (drawn < 0) {  // the last token with a nonzero probability
            int lp = -1;
            for (int j = 0; j < CH; ++j)
                if (gt[j] > 0.f) lp = i0 + j;
            for (int o = 32; o > 0; o >>= 1) lp = max(lp, __shfl_xor(lp, o));
            if ((t & 63) == 0) sh.redi[t >> 6] = lp;
            __syncthreads();
            drawn = sh.redi[0];
            for (int k = 1; k < kThreads / 64; ++k) drawn = max(drawn, sh.redi[k]);
            __syncthreads();
        }
        id = drawn;
    }
    if (id >= a.beg) tid = id;
    // the chosen token's probability and log probability, from its owner
    if (id >= i0 && id < i0 + ch) {
        const float x = vt[id - i0];
        const float p = gt[id - i0], plog = x > ninf ? __fsub_rn(x, ls) : ninf;
        if (out != nullptr) {
            out->p = p;
            out->plog = plog;
        }
        if (la.st != nullptr) {
            la.rec[lst.i].p = p;
            la.rec[lst.i].plog = plog;
        }
    }
    if (t == 0 && out != nullptr) {
        out->id = id;
        out->tid = tid;
        out->force_ts = force_ts;
        out->n_terms = terms;
    }
    if (t == 0 && la.st != nullptr) {
        // the loop's bookkeeping for this token (transcribe.go:211-237)
        const int i = lst.i;
        la.rec[i].id = id;
        la.rec[i].tid = tid;
        la.rec[i].force_ts = force_ts;
        lst.penult = lst.last;
        lst.last = id;
        ++lst.n_tokens;
        bool go = true;
        if (id > a.beg) {
            const int nd = 2 * (id - a.beg);
            if (lst.has_ts && lst.seek_delta > nd && lst.result_len < i) {
                lst.failed = 1;
                go = false;
            } else {
                lst.seek_delta = nd;
                lst.result_len = i + 1;
                lst.has_ts = 1;
            }
        }
        const bool at_end = la.seek + lst.seek_delta + la.delta_min >= la.seek_end;
        if (go && (id == a.eot || (lst.has_ts && at_end))) {
            if (lst.result_len == 0) {
                if (at_end) {
                    lst.result_len = i + 1;
                } else {
                    lst.failed = 1;
                    go = false;
                }
            }
            if (go) {
                lst.done = 1;
                go = false;
            }
        }
        if (go && i == la.n_max - 1 && (lst.result_len == 0 || lst.seek_delta < la.win_frames / 2))
            lst.failed = 1;  // stuck repeating itself
        lst.i = i + 1;
        *la.st = lst;
        *la.tok_w = id;
    }
}

template <int CH>
grx_status launch_ch(hipStream_t st, const float *logits, const GrxSampleArgs &a, const int *suppress, float *scratch,
                     GrxSampleOut *out, const GrxLoopArgs &la) {
    const size_t smem = sizeof(SampleShared);
    static bool attr = false;
    if (!attr) {
        if (hipFuncSetAttribute((const void *)sample_kernel<CH>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)smem) != hipSuccess)
            return grx_fail(GRX_EDEVICE, "whisper sampler: %zu bytes of LDS refused", smem);
        attr = true;
    }
    float *vg = scratch, *g = scratch + (size_t)kThreads * CH;
    sample_kernel<CH><<<1, kThreads, smem, st>>>(logits, a, suppress, vg, g, out, la);
    GRX_LAUNCHED("sample_kernel");
    return GRX_OK;
}

}  // namespace

grx_status grx_sample_launch(hipStream_t st, const float *logits, const GrxSampleArgs &a, const int *suppress,
                             float *scratch, GrxSampleOut *out, const GrxLoopArgs &la) {
    if (a.n <= 0 || a.n > kMaxLogits) return grx_fail(GRX_ESIZE, "whisper sampler: %d logits (1 .. %d)", a.n, kMaxLogits);
    const int per = (a.n + kThreads - 1) / kThreads;
    if (per <= 16) return launch_ch<16>(st, logits, a, suppress, scratch, out, la);
    if (per <= 32) return launch_ch<32>(st, logits, a, suppress, scratch, out, la);
    if (per <= 52) return launch_ch<52>(st, logits, a, suppress, scratch, out, la);
    return launch_ch<64>(st, logits, a, suppress, scratch, out, la);
}

grx_status grx_sample_args(const grx_whisper_rules *rules, const grx_whisper_seq *seq, int n, float temp, float r,
                           GrxSampleArgs *a) {
    if (!rules || !seq || !a || (rules->n_suppress > 0 && !rules->suppress) || rules->n_suppress < 0)
        return grx_fail(GRX_EINVAL, "whisper sampler: NULL argument");
    const grx_whisper_rules &v = *rules;
    for (int id : {v.eot, v.sot, v.translate, v.transcribe, v.solm, v.prev, v.nosp, v.no_timestamps, v.beg})
        if (id < 0 || id >= n) return grx_fail(GRX_EINVAL, "whisper sampler: token %d outside %d logits", id, n);
    if (v.n_lang < 0 || v.sot + v.n_lang >= n || v.space >= n || v.n_audio_ctx <= 0)
        return grx_fail(GRX_EINVAL, "whisper sampler: languages, space token or audio context out of range");
    *a = GrxSampleArgs{};
    a->n = n;
    a->eot = v.eot;
    a->sot = v.sot;
    a->not_ = v.no_timestamps;
    a->nosp = v.nosp;
    a->solm = v.solm;
    a->translate = v.translate;
    a->transcribe = v.transcribe;
    a->prev = v.prev;
    a->beg = v.beg;
    a->n_lang = v.n_lang;
    a->space = v.space;
    // transcribe.go:410-415: prec = 30/nAudioCtx, tid0 = round(maxInitialTS/prec)
    const double prec = 30.0 / (double)v.n_audio_ctx;
    a->tid0 = (int)round(v.max_initial_ts / prec);
    const int nt = seq->n_tokens;
    a->initial = nt == 0;
    a->last = nt > 0 && seq->last >= v.beg;
    a->penult = nt < 2 || seq->penult >= v.beg;
    a->has_ts = seq->has_ts != 0;
    a->seek_delta = seq->seek_delta;
    a->n_suppress = v.n_suppress;
    a->temp = temp;
    a->r = r;
    return GRX_OK;
}

grx_status grx_sample_run(grx_ctx *ctx, const float *dev_logits, const float *host_logits, int n,
                          const grx_whisper_rules *rules, const grx_whisper_seq *seq, float temp, float r,
                          grx_whisper_token *out) {
    if (!ctx || !out || (!dev_logits && !host_logits)) return grx_fail(GRX_EINVAL, "whisper sampler: NULL argument");
    GrxSampleArgs a;
    grx_status s = grx_sample_args(rules, seq, n, temp, r, &a);
    if (s != GRX_OK) return s;
    // ctx scratch: [result, 256 B][suppress list][logits and terms, 2 x 64k floats][host logits, copied]
    const size_t sbytes = ((size_t)a.n_suppress * 4 + 255) / 256 * 256, gbytes = (size_t)2 * 65536 * 4;
    const size_t lbytes = dev_logits ? 0 : (size_t)n * 4;
    void *buf;
    if ((s = grx_ctx_scratch(ctx, 256 + sbytes + gbytes + lbytes, &buf)) != GRX_OK) return s;
    float *dg = reinterpret_cast<float *>(static_cast<char *>(buf) + 256 + sbytes);
    GrxSampleOut *dout = static_cast<GrxSampleOut *>(buf);
    int *dsup = reinterpret_cast<int *>(static_cast<char *>(buf) + 256);
    const float *lg = dev_logits;
    GRX_HIP(hipSetDevice(ctx->device));
    hipStream_t st = ctx->stream;
    if (a.n_suppress > 0) GRX_HIP(hipMemcpyAsync(dsup, rules->suppress, (size_t)a.n_suppress * 4, hipMemcpyHostToDevice, st));
    if (!dev_logits) {
        float *dl = reinterpret_cast<float *>(static_cast<char *>(buf) + 256 + sbytes + gbytes);
        GRX_HIP(hipMemcpyAsync(dl, host_logits, lbytes, hipMemcpyHostToDevice, st));
        lg = dl;
    }
    if ((s = grx_sample_launch(st, lg, a, dsup, dg, dout)) != GRX_OK) return s;
    GrxSampleOut h;
    GRX_HIP(hipMemcpyAsync(&h, dout, sizeof h, hipMemcpyDeviceToHost, st));
    GRX_HIP(hipStreamSynchronize(st));
    out->id = h.id;
    out->tid = h.tid;
    out->p = h.p;
    out->plog = h.plog;
    out->force_ts = h.force_ts;
    return GRX_OK;
}

extern "C" grx_status grx_whisper_sample_logits(grx_ctx *ctx, const float *logits, int n, const grx_whisper_rules *rules,
                                                const grx_whisper_seq *seq, float temp, float r, grx_whisper_token *out) {
    if (!logits) return grx_fail(GRX_EINVAL, "grx_whisper_sample_logits: NULL logits");
    return grx_sample_run(ctx, nullptr, logits, n, rules, seq, temp, r, out);
}
