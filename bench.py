#!/usr/bin/env python3
"""Benchmark of the MI355X Q8_0 product (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload: the single Q8_0 GEMV shape (1024 x 1024, int8 U[-127,127], f16
scales |N(0,0.02)|/127, x ~ N(0,1) rounded to Q8_0 on the fly) over a ring of
512 distinct matrices (570 MB, more than the 256 MB Infinity Cache), so each
step streams every weight from HBM: one step = round x to Q8_0 + one GEMV
launch over all 512 matrices.  Inputs are resident in HBM before timing.

Prints one JSON line.  `value` is the whole-ring GEMV throughput in GB/s of
algorithmic bytes (34 B per 32 weights, plus x and y per matrix); `roofline`
is the GEMV kernel alone against 8 TB/s; `cpu_baseline` is the reference's
int8 route restated with VNNI intrinsics (oracle/grx_vnni.cc, bit-equal to
the oracle) on the same ring at one thread and at the host's threads.  Each
model loop's nested `cpu_baseline` runs the oracle's graph with its int8
products on that same kernel, at one thread and at the host's threads.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q8_0 GEMV GB/s (% HBM peak); decoder tokens/s at Whisper base.en shape"
HBM_PEAK_GBS = 8000.0
N, K, RING = 1024, 1024, 512
BYTES_PER_GEMV = N * K // 32 * 34 + K * 4 + N * 4   # 1,122,304 B per matrix


def measured_traffic() -> int | None:
    """HBM bytes per launch of the ring GEMV as rocprofv3's FETCH_SIZE and
    WRITE_SIZE counters read them, scaled by a copy of known size
    (profiles/gemv_q8_ring_traffic.txt, written from those runs)."""
    path = os.path.join(ROOT, "profiles", "gemv_q8_ring_traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes="):
            return int(line.split("=", 1)[1])
    return None


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="bound on the CPU baseline's work")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--decoder-steps", type=int, default=220,
                   help="greedy steps after the 4-token prompt (KV 4 -> 224)")
    p.add_argument("--no-decoder", action="store_true")
    p.add_argument("--lm-frames", type=int, default=250, help="pocket-TTS-style frames after the 64-row prefix")
    p.add_argument("--no-lm", action="store_true")
    p.add_argument("--streams-steps", type=int, default=220,
                   help="greedy steps of the 8-stream large-v3-turbo decoder after its 4-token prompt")
    p.add_argument("--no-streams", action="store_true")
    p.add_argument("--conformer-reps", type=int, default=10, help="timed encodes per batch size")
    p.add_argument("--no-conformer", action="store_true")
    p.add_argument("--no-conformer-stream", action="store_true")
    p.add_argument("--profile-leg", choices=["speak", "tdt", "sampler", "conformer-stream", "mimi"],
                   help="only this workload, for a profiler (no headline line): the pocket speak loop, the TDT "
                        "decode, whisper's sampler, the streaming chunk steps, or the Mimi decoder")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only copy the ring's bytes device to device 3 times (reference reading for HBM counters)")
    return p.parse_args()


def ring_weights(seed: int = 1) -> tuple[np.ndarray, np.ndarray]:
    """512 distinct 1024x1024 Q8_0 matrices stacked row-wise (one weight of
    524288 rows: each output row is that matrix's row, so one launch is 512
    GEMVs), and one activation vector."""
    from gorelaxor_amd.synth import q8_weight

    rng = np.random.default_rng(seed)
    w = q8_weight(rng, N * RING, K)
    x = rng.standard_normal(K).astype(np.float32)
    return w, x


def cpu_info() -> dict:
    """The host CPU: model name, logical CPUs, physical cores, the VNNI form
    the baseline takes."""
    model, phys = platform.processor() or platform.machine(), set()
    try:
        cur = {}
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                k, v = [t.strip() for t in line.split(":", 1)]
                cur[k] = v
                if k == "model name":
                    model = v
            elif cur:
                phys.add((cur.get("physical id"), cur.get("core id")))
                cur = {}
        if cur:
            phys.add((cur.get("physical id"), cur.get("core id")))
    except OSError:
        pass
    import oracle

    kind = {2: "AVX512-VNNI (EVEX)", 1: "AVX-VNNI (VEX)", 0: "none"}[oracle.vnni_kind()]
    return {"cpu": model, "logical_cpus": os.cpu_count(), "physical_cores": len(phys) or None, "vnni": kind}


def cpu_threads() -> int:
    """The host threads a baseline may use: the box's CPU share when it says
    (OMP_NUM_THREADS), else every logical CPU."""
    try:
        return max(1, int(os.environ.get("OMP_NUM_THREADS", "")))
    except ValueError:
        return os.cpu_count() or 1


def vnni_baseline(run, units: float, unit: str, sample: str) -> dict:
    """A model loop's CPU baseline: `run()` (a fresh oracle graph doing
    `units` of work; it returns the seconds of its timed part) with every
    int8 product on the reference's kernel restated with VNNI intrinsics
    (oracle/grx_vnni.cc: matmulQ8Int, quantU8avx, the 6x16 vpdpbusd tile,
    the reference's task split), at one thread and at the host's threads,
    each after an untimed run that packs every weight's panels (the
    reference's Pack on first use).  value: the all-thread rate.  The rest
    of the graph (attention, LayerNorm, the float routes) is the oracle's
    scalar C on one thread, where the reference would use its AVX2 kernels
    and fan some of it out, so the rate is a floor of the reference's."""
    import oracle

    th = cpu_threads()
    rates = {}
    for label, threads in (("one_thread", 1), ("all_threads", th)):
        with oracle.vnni_products(threads):
            run()
            rates[label] = units / run()
    return {"value": round(rates["all_threads"], 4), "unit": unit, "cores": th, "kind": "port", **cpu_info(),
            "one_thread": round(rates["one_thread"], 4), "threads": th,
            "sample": f"{sample}; int8 products on oracle/grx_vnni.cc (the reference's matmulQ8Int with VNNI) at "
                      f"1 and {th} threads, the rest scalar C on one thread"}


def cpu_baseline(w8: np.ndarray, x: np.ndarray, seconds: float) -> dict:
    """The reference's CPU path for the same products: matmulQ8Int with the
    VNNI tile kernel and its task split (internal/kern/q8int.go:148-223,
    vnni_amd64.s), restated with intrinsics in oracle/grx_vnni.cc and
    checked bit-equal to the oracle; one kern.MatMul per matrix of the same
    512-matrix ring, at all of the box's threads (`value`) and at one, plus
    one matrix over and over (cache-resident, as the reference's own kernel
    benchmark runs it).  GB/s of the same algorithmic bytes."""
    import oracle

    oracle.build()
    info = cpu_info()
    if oracle.vnni_kind() == 0:
        return {"value": None, "unit": "GB/s", "cores": 0, "kind": "port", **info,
                "sample": "this CPU has neither AVX512-VNNI nor AVX-VNNI: the reference's int8 kernel cannot run"}
    panels, per = oracle.vnni_pack_many(w8, RING, N, K)
    y = np.zeros(RING * N, np.float32)
    want = oracle.matmul_q8_int(x, w8[:N * K // 32 * 34], N, K)[0]
    oracle.vnni_ring(y, x, panels, per, 1, N, K, 1, 1)
    same = bool(np.array_equal(y[:N].view(np.uint32), want.view(np.uint32)))
    budget = seconds / 8

    def rate(count: int, threads: int) -> tuple[float, int]:
        # one pass to size the sample, then whole passes filling the budget
        t0 = time.perf_counter()
        oracle.vnni_ring(y, x, panels, per, count, N, K, threads, 1)
        one = time.perf_counter() - t0
        reps = max(1, int(budget / max(one, 1e-6)))
        t0 = time.perf_counter()
        oracle.vnni_ring(y, x, panels, per, count, N, K, threads, reps)
        el = time.perf_counter() - t0
        return reps * count * BYTES_PER_GEMV / el / 1e9, reps * count

    th = cpu_threads()
    # the ring at every power-of-two thread count up to the host's: for one
    # row of 1024 x 1024 the task split's hand-offs can cost more than the
    # extra threads bring, so `value` is the best count's rate
    sweep = {}
    t = 1
    while True:
        sweep[t] = rate(RING, t)
        if t >= th:
            break
        t = min(2 * t, th)
    best_th = max(sweep, key=lambda k: sweep[k][0])
    single_all, _ = rate(1, th)
    single_one, _ = rate(1, 1)
    return {"value": round(sweep[best_th][0], 3), "unit": "GB/s", "cores": best_th, "kind": "port", **info,
            "parity_bit_exact": same,
            "ring": {"threads": th, "value": round(sweep[th][0], 3), "one_thread": round(sweep[1][0], 3),
                     "by_threads": {str(k): round(v[0], 3) for k, v in sweep.items()}, "unit": "GB/s"},
            "cache_resident_single_matrix": {"threads": th, "value": round(single_all, 3),
                                             "one_thread": round(single_one, 3), "unit": "GB/s"},
            "sample": f"{sweep[best_th][1]} GEMVs of 1024x1024 over the 512-matrix ring at {best_th} thread(s) (the "
                      f"best of {sorted(sweep)}), about {budget:.1f} s each, oracle/grx_vnni.cc (matmulQ8Int, "
                      f"quantU8avx, q8tile with vpdpbusd, the reference's task split)"}


PROMPT = [50257, 50362, 50363, 50258]


def whisper_step_bytes(hp: dict, streams: int, positions) -> dict:
    """Algorithmic HBM bytes of one decoder step, averaged over the steps'
    positions: the Q8_0 matrices the step multiplies (per layer: self-
    attention q|k|v and out, cross query and out, fc1, fc2; the token
    embedding as the logits matrix; the cross keys and values were
    projected once per window), every stream's cross keys and values
    (float32), and the self-attention cache rows up to the position."""
    d, nl, nv, na = hp["n_state"], hp["n_layer"], hp["n_vocab"], hp["n_audio_ctx"]
    ff = 4 * d
    weights = (nl * (6 * d * d + 2 * ff * d) + nv * d) // 32 * 34
    cross = streams * nl * 2 * na * d * 4
    self_kv = streams * nl * 2 * d * 4 * float(np.mean([p + 1 for p in positions]))
    return {"weights": weights, "cross_kv": cross, "self_kv_avg": int(self_kv),
            "total": int(weights + cross + self_kv)}


def roofline(bytes_per_step: float, s_per_step: float) -> dict:
    gbs = bytes_per_step / s_per_step / 1e9
    return {"bound": "hbm", "bytes_per_step": int(bytes_per_step), "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)}


def decoder_bench(args) -> dict:
    """whisper base.en-shaped decoder with random-init Q8_0 weights: cross
    attention over a 1500 x 512 N(0,1) encoder output, a 4-token prompt, then
    `decoder_steps` greedy steps (KV 4 -> 224), all on the device.  Reports
    decoder steps per second (one token through the decoder per step), and
    checks the tokens against the oracle's."""
    import oracle
    from gorelaxor_amd.synth import WHISPER_BASE_EN, encoder_output, whisper_model
    from gorelaxor_amd.whisper import WhisperDecoder

    hp = dict(WHISPER_BASE_EN)
    t = whisper_model(hp, seed=7)
    enc = encoder_output(hp, seed=8)
    dec = WhisperDecoder(hp, t)
    t0 = time.perf_counter()
    dec.set_encoder_output(enc)  # the first call also sends the weights to the device
    first_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    dec.set_encoder_output(enc)  # a later window: the cross keys and values alone
    cross_s = time.perf_counter() - t0
    n = args.decoder_steps
    dec.greedy(PROMPT, n)  # warm: graph captured, caches warm
    reps = 3
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        toks = dec.greedy(PROMPT, n)
        times.append(time.perf_counter() - t0)
    best = min(times)
    steps = len(PROMPT) + n
    sb = whisper_step_bytes(hp, 1, range(steps))
    res = {"tokens_per_s": round(steps / best, 1), "ms_per_token": round(best / steps * 1e3, 4),
           "steps_per_run": steps, "generated_tokens": n + 1, "runs": reps,
           "roofline": roofline(sb["total"], best / steps), "step_bytes": sb,
           "cross_kv_ms_per_window": round(cross_s * 1e3, 2), "first_window_ms_with_weight_upload": round(first_s * 1e3, 2),
           "shape": "d_model 512, 8 heads, 6 layers, FFN 2048, vocab 51864, audio 1500, KV 4->%d" % (len(PROMPT) + n)}
    oracle.build()
    ref = oracle.WhisperOracle(hp, t)
    ref.set_encoder_output(enc)
    t0 = time.perf_counter()
    want = ref.greedy(PROMPT, n)
    cpu_s = time.perf_counter() - t0
    res["parity_tokens_identical"] = bool(np.array_equal(want, toks))

    def run_dec():
        r = oracle.WhisperOracle(hp, t)
        r.set_encoder_output(enc)
        t0 = time.perf_counter()
        r.greedy(PROMPT, n)
        return time.perf_counter() - t0

    res["cpu_baseline"] = vnni_baseline(run_dec, steps, "tokens/s", f"the same {steps} decoder steps on the oracle")
    res["cpu_baseline"]["scalar_one_thread"] = round(steps / cpu_s, 2)
    if not args.no_cpu:
        res["cpu_reference_f16"] = f16_decode_baseline(ref, t, n, steps)
    res["rules_loop"] = rules_loop_bench(dec, ref, n)
    dec.close()
    return res


def rules_loop_bench(dec, ref, n: int) -> dict:
    """The window loop with whisper's token rules on the device
    (grx_whisper_rules_loop: process + sample on each step's logits, the
    loop's timestamp and end rules, the token fed back, no host round trip)
    after the 4-token prompt, `n` iterations at temperature 0 with the
    timestamp tokens in the suppress list (so the random-init model's loop
    runs all n iterations), against the oracle's restatement of the same
    loop: every token's id, best timestamp and the bits of p and plog."""
    import oracle
    from gorelaxor_amd.whisper import Rules, special_tokens

    hp = dec.hp
    sp = special_tokens(hp["n_vocab"])
    sup = [1, 2, 7, 8, 9, 10, 220, 1906, 3556, 50254] + list(range(sp["beg"], hp["n_vocab"]))
    rules = Rules(sp, sup, space=220)
    times = []
    for _ in range(3):
        dec.reset()
        t0 = time.perf_counter()
        dec.decode(PROMPT, want_logits=False)
        got, st = dec.rules_loop(rules, 0, 30000, n)
        times.append(time.perf_counter() - t0)
    best = min(times)
    steps = len(PROMPT) + st["n_tokens"]
    ref.reset()
    lr = ref.decode(PROMPT)
    t0 = time.perf_counter()
    want, wst = oracle.whisper_window_loop(ref, lr, sp, suppress=sup, space=220, seek=0, seek_end=30000, n_max=n)
    cpu_s = time.perf_counter() - t0

    def same(g, w):
        return (g["id"], g["tid"]) == (w["id"], w["tid"]) and all(
            np.float32(g[k]).view(np.uint32) == np.float32(w[k]).view(np.uint32) for k in ("p", "plog"))

    ok = st == wst and len(got) == len(want) and all(same(g, w) for g, w in zip(got, want))
    return {"tokens_per_s": round(steps / best, 1), "ms_per_token": round(best / steps * 1e3, 4),
            "iterations": st["n_tokens"], "parity_bit_exact": bool(ok),
            "cpu_baseline": {"value": round(st["n_tokens"] / cpu_s, 2), "unit": "tokens/s", "cores": 1,
                             "kind": "port", **cpu_info(),
                             "sample": f"the same {st['n_tokens']} iterations of the oracle's loop (decode and "
                                       f"sampler, scalar C, 1 thread), {cpu_s:.2f} s"}}


def f16_decode_baseline(ref, t, n: int, steps: int) -> dict:
    """The reference's own whisper decode on the host (float16 matrices, its
    AVX2/F16C kernels and thread fan-out, oracle/grx_vnni.cc f16w_decode
    restating whisper/decoder.go and gemm.go:223-256) over the same prompt
    and steps, at one thread and at the host's threads: tokens/s.  Its
    matrices are the Q8_0 ones widened to float16, so its tokens are its
    own; this is the rate a user of the reference gets today."""
    import oracle

    f16 = oracle.WhisperF16(ref, t)
    out = {"unit": "tokens/s", "kind": "port", **cpu_info()}
    th = cpu_threads()
    for label, threads in (("one_thread", 1), ("all_threads", th)):
        f16.reset()
        t0 = time.perf_counter()
        f16.greedy(PROMPT, n, threads)
        out[label] = round(steps / (time.perf_counter() - t0), 2)
    out["threads"] = th
    out["sample"] = (f"the same {steps} decoder steps (4-token prompt in one call, then one token a step) on "
                     f"float16 matrices, at 1 and {th} threads")
    return out


def streams_bench(args) -> dict:
    """whisper large-v3-turbo-shaped decoder with random-init Q8_0 weights (d
    1280, 20 heads, 4 layers, FFN 5120, vocab 51866), 8 independent streams
    each with its own 1500 x 1280 N(0,1) encoder output, stepping together
    (every product 8 rows): 4-token prompt + `streams_steps` greedy steps
    per stream.  Aggregate tokens/s over the 8 streams; stream 0's tokens
    checked against the oracle (whose rate on that stream is the CPU
    baseline; the reference decodes one stream at a time) and stream 3's
    against its own single-stream decode on the GPU."""
    import oracle
    from gorelaxor_amd.synth import WHISPER_LARGE_V3_TURBO, encoder_output, whisper_model
    from gorelaxor_amd.whisper import WhisperDecoder

    hp = dict(WHISPER_LARGE_V3_TURBO)
    S, n = 8, args.streams_steps
    t = whisper_model(hp, seed=23)
    encs = [encoder_output(hp, seed=60 + k) for k in range(S)]
    dec = WhisperDecoder(hp, t, streams=S)
    dec.set_encoder_output_stream(0, encs[0])  # the first call also sends the weights to the device
    t0 = time.perf_counter()
    for k in range(S):
        dec.set_encoder_output_stream(k, encs[k])
    cross_s = time.perf_counter() - t0
    prompt = [PROMPT] * S
    dec.greedy_streams(prompt, n)  # warm: graph captured
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        toks = dec.greedy_streams(prompt, n)
        times.append(time.perf_counter() - t0)
    best = min(times)
    steps = len(PROMPT) + n
    sb = whisper_step_bytes(hp, S, range(steps))
    res = {"tokens_per_s": round(S * steps / best, 1), "ms_per_step": round(best / steps * 1e3, 4),
           "streams": S, "steps_per_run": steps, "runs": 3,
           "roofline": roofline(sb["total"], best / steps), "step_bytes": sb,
           "cross_kv_ms_all_streams": round(cross_s * 1e3, 1),
           "shape": "d_model 1280, 20 heads, 4 layers, FFN 5120, vocab 51866, audio 1500, 8 streams, KV 4->%d"
                    % steps}
    dec.close()
    one = WhisperDecoder(hp, t)
    one.set_encoder_output(encs[3])
    same = bool(np.array_equal(one.greedy(PROMPT, n), toks[3]))
    one.close()
    oracle.build()
    ref = oracle.WhisperOracle(hp, t)
    ref.set_encoder_output(encs[0])
    t0 = time.perf_counter()
    want = ref.greedy(PROMPT, n)
    cpu_s = time.perf_counter() - t0
    res["parity_tokens_identical"] = bool(np.array_equal(want, toks[0])) and same
    ns = 32  # decoder steps timed (bounded sample)

    def run_streams():
        r = oracle.WhisperOracle(hp, t)
        r.set_encoder_output(encs[0])
        t0 = time.perf_counter()
        r.greedy(PROMPT, ns)
        return time.perf_counter() - t0

    res["cpu_baseline"] = vnni_baseline(run_streams, len(PROMPT) + ns, "tokens/s",
                                        f"stream 0's first {len(PROMPT) + ns} decoder steps on the oracle (the "
                                        f"reference decodes streams one after another)")
    res["cpu_baseline"]["scalar_one_thread"] = round(steps / cpu_s, 2)
    return res


def lm_bench(args) -> dict:
    """pocket-TTS-style flow-LM transformer with random-init Q8_0 weights (d
    1024, 16 heads, 6 layers, FFN 4096): a 64-row random-embedding text
    prefix, then `lm_frames` teacher-forced latent frames (KV 64 -> 314),
    all on the device; frames per second, outputs checked against the
    oracle's, which is also the CPU baseline."""
    import oracle
    from gorelaxor_amd.pocket import PocketLM
    from gorelaxor_amd.synth import POCKET_TTS_LM, pocket_inputs, pocket_model

    hp = dict(POCKET_TTS_LM)
    n = args.lm_frames
    t = pocket_model(hp, seed=5)
    x, lat = pocket_inputs(hp, n, prefix=64, seed=6)
    lm = PocketLM(hp, t)
    lm.run(x)
    lm.frames(lat)  # warm: graph captured, caches warm
    reps, times = 3, []
    for _ in range(reps):
        lm.reset()
        t0 = time.perf_counter()
        lm.run(x)
        t1 = time.perf_counter()
        outs, eos = lm.frames(lat)
        times.append((t1 - t0, time.perf_counter() - t1))
    prefix_s = min(a for a, _ in times)
    frames_s = min(b for _, b in times)
    # per frame: the Q8_0 matrices (per layer q|k|v, out, ff1, ff2), the
    # float32 input projection, out_norm and eos vectors, and the cache rows
    # up to the frame's position (the 64-row prefix first)
    d, ff, nl, ld = hp["d"], hp["ff"], hp["n_layer"], hp["ldim"]
    wq8 = nl * (4 * d * d + 2 * ff * d) // 32 * 34
    small = (ld * d + 5 * d) * 4
    kv = nl * 2 * d * 4 * float(np.mean([64 + f + 1 for f in range(n)]))
    frame_bytes = wq8 + small + kv
    res = {"frames_per_s": round(n / frames_s, 1), "ms_per_frame": round(frames_s / n * 1e3, 4),
           "roofline": roofline(frame_bytes, frames_s / n),
           "frame_bytes": {"weights": wq8, "vectors": small, "kv_avg": int(kv), "total": int(frame_bytes)},
           "prefix_ms": round(prefix_s * 1e3, 3), "prefix_int8_tops": round(
               2 * 64 * nl * (4 * d * d + 2 * ff * d) / prefix_s / 1e12, 2),
           "frames": n, "prefix_rows": 64, "runs": reps,
           "shape": "d_model 1024, 16 heads, 6 layers, FFN 4096, KV 64->%d" % (64 + n)}
    oracle.build()
    ref = oracle.PocketOracle(hp, t)
    t0 = time.perf_counter()
    ref.run(x)
    t1 = time.perf_counter()
    ok = True
    for k in range(n):
        wo, we = ref.step(lat[k])
        ok = ok and bool(np.array_equal(wo.view(np.uint32), outs[k].view(np.uint32))) and bool(np.float32(we) == eos[k])
    cpu_s = time.perf_counter() - t1
    res["parity_bit_exact"] = ok
    nf = 40  # frames timed (bounded sample)

    def run_lm():
        r = oracle.PocketOracle(hp, t)
        r.run(x)
        t0 = time.perf_counter()
        for k in range(nf):
            r.step(lat[k])
        return time.perf_counter() - t0

    res["cpu_baseline"] = vnni_baseline(run_lm, nf, "frames/s", f"the first {nf} frames after the 64-row prefix on the oracle")
    res["cpu_baseline"]["scalar_one_thread"] = round(n / cpu_s, 2)
    lm.close()
    res["speak"] = speak_bench(args, hp, t, x)
    res["mimi"] = mimi_bench(args)
    return res


def speak_bench(args, hp, t, x) -> dict:
    """speakChunk's frame loop on the device: per frame the transformer step
    fed the previous sampled latent, then the flow head (512 wide, 6
    residual blocks, 1 LSD step, random-init, typed as converted files:
    Q8_0 matrices on kern's float route, float32 input/output projections)
    from its output and seeded noise; frames per second, latents checked
    against the oracle's."""
    import oracle
    from gorelaxor_amd.pocket import PocketLM
    from gorelaxor_amd.synth import POCKET_FLOW, pocket_flow_model

    fhp = dict(POCKET_FLOW)
    n = args.lm_frames
    ft = pocket_flow_model(hp, fhp, seed=7)
    noise = np.random.default_rng(8).standard_normal((n, hp["ldim"])).astype(np.float32) * np.float32(0.3 ** 0.5)
    lm = PocketLM(hp, t)
    lm.flow_init(fhp["dim"], fhp["depth"], fhp["steps"])
    for k, v in ft.items():
        lm.set_tensor(k, v)
    lm.run(x)
    lm.speak(noise)  # warm: graph captured
    times = []
    for _ in range(3):
        lm.reset()
        lm.run(x)
        t0 = time.perf_counter()
        lats, eos = lm.speak(noise)
        times.append(time.perf_counter() - t0)
    lm.close()
    best = min(times)
    res = {"frames_per_s": round(n / best, 1), "ms_per_frame": round(best / n * 1e3, 4), "frames": n,
           "flow_head": "dim %d, %d residual blocks, %d LSD step(s)" % (fhp["dim"], fhp["depth"], fhp["steps"])}
    oracle.build()
    ref = oracle.PocketOracle(hp, t)
    flow = oracle.PocketFlowOracle(hp, fhp["dim"], fhp["depth"], fhp["steps"], ft)
    ref.run(x)
    ok, latent = True, None
    t0 = time.perf_counter()
    for k in range(n):
        h, e = ref.step(latent)
        latent = flow.sample(h, noise[k])
        ok = ok and bool(np.array_equal(latent.view(np.uint32), lats[k].view(np.uint32))) and \
            bool(np.float32(e) == eos[k])
    scalar = n / (time.perf_counter() - t0)
    res["parity_bit_exact"] = ok
    nf = 30

    def run_speak():
        r = oracle.PocketOracle(hp, t)
        r.run(x)
        lt = None
        t0 = time.perf_counter()
        for k in range(nf):
            h, _ = r.step(lt)
            lt = flow.sample(h, noise[k])
        return time.perf_counter() - t0

    res["cpu_baseline"] = vnni_baseline(run_speak, nf, "frames/s",
                                        f"the first {nf} frames (transformer step and flow head, Python glue) on "
                                        f"the oracle")
    res["cpu_baseline"]["scalar_one_thread"] = round(scalar, 2)
    return res


def mimi_bench(args) -> dict:
    """Pocket TTS's Mimi decoder at the english_2026-09 shape (d 512, 8
    heads, 2 layers, context 250, 16x upsampling, SEANet 6/5/4: 1920
    samples at 24 kHz per latent), random-init with the converter's typing,
    decoding lm_frames latents one per call as the speak loop does (a host
    round trip each): latents/s and the real-time factor; the first 8
    latents checked bit for bit against the oracle, whose rate is the CPU
    baseline."""
    import oracle
    from gorelaxor_amd.mimi import MimiDecoder
    from gorelaxor_amd.synth import MIMI, mimi_latents, mimi_model

    hp = dict(MIMI)
    n = args.lm_frames
    t = mimi_model(hp, seed=17)
    lat = mimi_latents(hp, n, seed=18)
    dec = MimiDecoder(hp, t, max_latents=1)
    spl = dec.samples_per_latent
    first = np.concatenate([dec.decode(lat[k:k + 1]) for k in range(8)])
    times = []
    for _ in range(3):
        dec.reset()
        t0 = time.perf_counter()
        for k in range(n):
            dec.decode(lat[k:k + 1])
        times.append(time.perf_counter() - t0)
    dec.close()
    best = min(times)
    audio_s = n * spl / 24000.0
    res = {"latents_per_s": round(n / best, 1), "ms_per_latent": round(best / n * 1e3, 4), "latents": n,
           "samples_per_latent": spl, "real_time_factor": round(audio_s / best, 1),
           "shape": "d_model 512, 8 heads, 2 layers, FFN 2048, context 250, upsample 16, SEANet ratios 6/5/4, "
                    "64 filters"}
    oracle.build()
    ref = oracle.MimiOracle(hp, t)
    t0 = time.perf_counter()
    want = np.concatenate([ref.decode(lat[k:k + 1]) for k in range(8)])
    cpu_s = time.perf_counter() - t0
    res["parity_first_8_bit_exact"] = bool(np.array_equal(want.view(np.uint32), first.view(np.uint32)))

    def run_mimi():
        r = oracle.MimiOracle(hp, t)
        t0 = time.perf_counter()
        for k in range(8):
            r.decode(lat[k:k + 1])
        return time.perf_counter() - t0

    res["cpu_baseline"] = vnni_baseline(run_mimi, 8, "latents/s", "the first 8 latents on the oracle, one per call")
    res["cpu_baseline"]["scalar_one_thread"] = round(8 / cpu_s, 2)
    return res


MFMA_INT8_PEAK_TOPS = 5000.0   # MI355X dense int8 matrix peak, 5.0 POP/s


def conformer_ops(hp: dict, frames: int, batch: int) -> int:
    """Algorithmic int8 operations (2 per multiply-add) of every Linear of
    one encode of `batch` utterances of `frames` mel frames: the
    pre-encoder's two pointwise products and its output product, each
    block's feed-forward, q|k|v, out and pointwise products on batch*T rows,
    and each block's position projection on 2T-1 rows (shared)."""
    d, c, ff, nl = hp["d"], hp["sub_channels"], hp["dff"], hp["layers"]
    so = lambda n: (n - 1) // 2 + 1  # noqa: E731
    T1, T2, T = so(frames), so(so(frames)), so(so(so(frames)))
    F2, F3 = so(so(hp["n_mels"])), so(so(so(hp["n_mels"])))
    pre = T2 * F2 * c * c + T * F3 * c * c + T * d * c * F3
    per_row = 4 * ff * d + 3 * d * d + d * d + 2 * d * d + d * d
    return 2 * (batch * (pre + nl * T * per_row) + nl * (2 * T - 1) * d * d)


def conformer_weight_bytes(hp: dict) -> int:
    """Q8_0 bytes of every Linear weight of the encoder (34 per 32)."""
    d, c, ff, nl = hp["d"], hp["sub_channels"], hp["dff"], hp["layers"]
    so = lambda n: (n - 1) // 2 + 1  # noqa: E731
    F3 = so(so(so(hp["n_mels"])))
    vals = 2 * c * c + d * c * F3 + nl * (4 * ff * d + 5 * d * d + 2 * d * d + d * d)
    return vals // 32 * 34


def conformer_bench(args) -> dict:
    """Parakeet-TDT-0.6B-shaped FastConformer encoder forward (d 1024, 24
    layers, FFN 4096, 8 heads, kernel 31, 256 pre-encoder channels) with
    random-init Q8_0 weights over 10 s of white noise (N(0, 0.1^2), 16 kHz)
    as 128-bin log-mel (1001 frames -> 126 encoder frames, 125 valid), at
    batch 1 and 16, mel and output resident in HBM.  Utterances/s, int8 TOPS
    of the Linears against the 5 POP/s MFMA peak; batch 1 output checked
    against the oracle, whose encode of the same utterance is the CPU
    baseline, and each utterance of the batch of 16 against its own batch-1
    encode."""
    import oracle
    from gorelaxor_amd import hiprt
    from gorelaxor_amd.conformer import ConformerEncoder, frames_out
    from gorelaxor_amd.synth import PARAKEET_TDT_06B, conformer_model, noise_mel

    hp = dict(PARAKEET_TDT_06B)
    t = conformer_model(hp, seed=32)
    mels = [noise_mel(hp["n_mels"], 10.0, seed=70 + i) for i in range(16)]
    frames, valid = mels[0][1], mels[0][2]
    mel = np.stack([m for m, _, _ in mels])
    T = frames_out(frames)
    enc = ConformerEncoder(hp, t)
    stream = enc.ctx.stream
    res = {"shape": "d_model 1024, 24 layers, FFN 4096, 8 heads, conv kernel 31, 128 mels, 10 s -> T %d" % T}
    d = hp["d"]
    for batch in (1, 16):
        dm = hiprt.DeviceBuffer.from_array(np.ascontiguousarray(mel[:batch]))
        do = hiprt.DeviceBuffer(batch * T * d * 4)
        enc.encode_dev(dm.ptr, batch, frames, valid, do.ptr)  # plan + capture
        enc.encode_dev(dm.ptr, batch, frames, valid, do.ptr)
        ms = []
        for _ in range(args.conformer_reps):
            a, b = hiprt.Event(), hiprt.Event()
            a.record(stream)
            enc.encode_dev(dm.ptr, batch, frames, valid, do.ptr)
            b.record(stream)
            b.synchronize()
            ms.append(a.elapsed_ms(b))
        best = float(np.median(ms))
        ops = conformer_ops(hp, frames, batch)
        r = {"utterances_per_s": round(batch / (best * 1e-3), 2), "ms_per_encode": round(best, 3),
             "int8_tops": round(ops / (best * 1e-3) / 1e12, 2), "int8_ops_per_encode": ops,
             "mfma_fraction": round(ops / (best * 1e-3) / 1e12 / MFMA_INT8_PEAK_TOPS, 4), "reps": args.conformer_reps}
        if batch == 1:
            wbytes = conformer_weight_bytes(hp)
            r["weight_bytes"] = wbytes
            r["weight_stream_gbs"] = round(wbytes / (best * 1e-3) / 1e9, 1)
            out1 = do.download(np.float32, (T, d))
        else:
            out16 = do.download(np.float32, (batch, T, d))
        res[f"batch{batch}"] = r
        del dm, do
    # each utterance of the batch of 16 bit-identical to its own batch-1
    # encode (utterance 0's batch-1 encode is checked against the oracle)
    same16 = True
    for i in range(16):
        one, _ = enc.encode(mel[i:i + 1], valid)
        same16 = same16 and bool(np.array_equal(one[0].view(np.uint32), out16[i].view(np.uint32)))
    same16 = same16 and bool(np.array_equal(out1.view(np.uint32), out16[0].view(np.uint32)))
    enc.close()
    oracle.build()
    t0 = time.perf_counter()
    want, L = oracle.ConformerOracle(hp, t).encode(mel[0], valid)
    cpu_s = time.perf_counter() - t0
    res["parity_bit_exact"] = bool(np.array_equal(out1.view(np.uint32), want.view(np.uint32)))
    res["batch16"]["parity_each_equals_its_batch1_encode"] = same16
    def run_conf():
        o = oracle.ConformerOracle(hp, t)
        t0 = time.perf_counter()
        o.encode(mel[0], valid)
        return time.perf_counter() - t0

    res["cpu_baseline"] = vnni_baseline(run_conf, 1.0, "utterances/s",
                                        "one 10 s utterance, all 24 layers, on the oracle")
    res["cpu_baseline"]["scalar_one_thread"] = round(1.0 / cpu_s, 4)
    res["tdt_decode"] = tdt_bench(args, want[:L])
    return res


def stream_step_bytes(hp: dict, weight_bytes: int, batch: int, keys: int, rows: int) -> int:
    """HBM bytes of one chunk step: every Linear weight once (Q8_0), and per
    stream and layer the keys and values its queries read (keys rows of 2d
    float32), the chunk's own rows written into the rings, and the
    convolution cache read and written (pad_left rows of d)."""
    d, nl = hp["d"], hp["layers"]
    pl = hp["conv_left"] if hp.get("conv_left", -1) >= 0 and hp.get("conv_right", -1) >= 0 else \
        (hp["conv_kernel"] - 1) // 2
    per = nl * (keys * 2 * d * 4 + rows * 2 * 2 * d * 4 + 2 * pl * d * 4)
    return weight_bytes + batch * per


def conformer_stream_bench(args) -> dict:
    """Cache-aware streaming (conformer/stream.go:241-307) of a
    Nemotron-Speech-Streaming-shaped encoder (d 1024, 24 layers, FFN 4096,
    8 heads, causal convolution of 9 taps, 70 rows of left context) with
    random-init Q8_0 weights over 10 s of white noise: every chunk step of
    the recording at right context 13 (chunks of 14 rows, 1.12 s of audio)
    and 0 (one row, 80 ms), for 1 and 16 streams stepped together, chunk
    mels resident in HBM.  ms per chunk step (the API call, which waits for
    its output), encoder rows/s, real-time factor, HBM bytes per step and
    their roofline; the first chunks checked against the oracle, whose
    chunk steps are the CPU baseline."""
    import oracle
    from gorelaxor_amd import hiprt
    from gorelaxor_amd.conformer import ConformerEncoder, ConformerStream, mel_chunks, stream_geom
    from gorelaxor_amd.synth import NEMOTRON_STREAMING, conformer_model, noise_mel

    hp = dict(NEMOTRON_STREAMING)
    t = conformer_model(hp, seed=35)
    mels = [noise_mel(hp["n_mels"], 10.0, seed=90 + i)[0] for i in range(16)]
    enc = ConformerEncoder(hp, t)
    d = hp["d"]
    c, F3 = hp["sub_channels"], hp["n_mels"]
    for _ in range(3):
        F3 = F3 // 2 + 1
    wbytes = (2 * c * c + d * c * F3 + hp["layers"] * (4 * hp["dff"] * d + 5 * d * d + 2 * d * d + d * d)) // 32 * 34
    res = {"shape": "d_model 1024, 24 layers, FFN 4096, 8 heads, causal conv kernel 9, 128 mels, left context 70",
           "weight_bytes": wbytes}
    oracle.build()
    for right in (13, 0):
        g = stream_geom(hp, right)
        chunks = [mel_chunks(m, g) for m in mels]
        n = len(chunks[0])
        r = {"chunk_rows": g["chunk"], "chunk_audio_s": g["mel_next"] * 0.01, "chunks": n}
        for batch in (1, 16):
            s = ConformerStream(enc, right, batch=batch)
            dms = [hiprt.DeviceBuffer.from_array(np.ascontiguousarray(np.stack([chunks[b][j][0] for b in range(batch)])))
                   for j in range(n)]
            do = hiprt.DeviceBuffer(batch * g["chunk"] * d * 4)
            times, first_rows = [], None
            for j in range(n):
                nf = chunks[0][j][0].shape[1]
                t0 = time.perf_counter()
                s.step_dev(dms[j].ptr, nf, [chunks[b][j][1] for b in range(batch)], do.ptr)
                times.append(time.perf_counter() - t0)
                if j < 2 and batch == 1:
                    first_rows = (first_rows or []) + [do.download(np.float32, (g["chunk"], d))]
            s.close()
            del dms, do
            # the steady chunks: the left context full, every graph captured
            steady = [x for j, x in enumerate(times) if j >= 2 and chunks[0][j][0].shape[1] == chunks[0][2][0].shape[1]]
            ms = float(np.median(steady)) * 1e3
            keys = g["left"] + g["chunk"]
            sb = stream_step_bytes(hp, wbytes, batch, keys, g["chunk"])
            r[f"batch{batch}"] = {"ms_per_chunk": round(ms, 3),
                                  "rows_per_s": round(batch * g["chunk"] / (ms * 1e-3), 1),
                                  "real_time_factor": round(batch * g["mel_next"] * 0.01 / (ms * 1e-3), 1),
                                  "step_bytes": sb, "roofline": roofline(sb, ms * 1e-3),
                                  "first_chunk_ms": round(times[0] * 1e3, 3)}
            if batch == 1:
                o = oracle.ConformerOracle(hp, t).stream(right, g["left"], g["drop"])
                same, cpu = True, []
                for j in range(2):
                    ch, ln, _ = chunks[0][j]
                    t0 = time.perf_counter()
                    want = o.step(ch, ln)
                    cpu.append(time.perf_counter() - t0)
                    got = first_rows[j][:len(want)]
                    same = same and bool(np.array_equal(got.view(np.uint32), want.view(np.uint32)))
                r["parity_first_chunks_bit_exact"] = same

                def run_chunk(right=right, g=g):
                    o2 = oracle.ConformerOracle(hp, t).stream(right, g["left"], g["drop"])
                    ch0, ln0, _ = chunks[0][0]
                    o2.step(ch0, ln0)
                    ch1, ln1, _ = chunks[0][1]
                    t0 = time.perf_counter()
                    o2.step(ch1, ln1)
                    return time.perf_counter() - t0

                r["cpu_baseline"] = vnni_baseline(run_chunk, 1.0, "chunk steps/s",
                                                  "the second chunk step of one stream on the oracle")
                r["cpu_baseline"]["scalar_one_thread"] = round(1.0 / cpu[1], 3)
        res[f"right{right}"] = r
    enc.close()
    return res


def tdt_bench(args, enc: np.ndarray) -> dict:
    """Model.Decode's greedy TDT loop (conformer/rnnt.go:111-173) over the
    encoder output of the 10 s utterance, with a Parakeet-TDT-shaped head
    (2 x 640 LSTM, joint 640, 1024 tokens + blank, durations 0..4,
    random-init Q8_0): the whole loop on the device, encoder output resident
    in HBM; decodes per second and tokens, checked against the oracle, whose
    decode is the CPU baseline."""
    import oracle
    from gorelaxor_amd import hiprt
    from gorelaxor_amd.rnnt import TransducerDecoder
    from gorelaxor_amd.synth import RNNT_TDT, rnnt_model

    hp = dict(RNNT_TDT)
    t = rnnt_model(hp, seed=33)
    T = enc.shape[0]
    dec = TransducerDecoder(hp, t)
    de = hiprt.DeviceBuffer.from_array(np.ascontiguousarray(enc, np.float32))
    got = dec.decode_dev(de.ptr, T)  # graph captured
    times = []
    for _ in range(args.conformer_reps):
        t0 = time.perf_counter()
        dec.decode_dev(de.ptr, T)
        times.append(time.perf_counter() - t0)
    dec.close()
    del de
    best = float(np.median(times))
    oracle.build()
    t0 = time.perf_counter()
    want, _ = oracle.RnntOracle(hp, t).decode(enc)
    cpu_s = time.perf_counter() - t0
    same = len(got) == len(want) and all(
        (g.ID, g.Frame, g.Duration) == w[:3] and np.float32(g.P).tobytes() == np.float32(w[3]).tobytes()
        for g, w in zip(got, want))

    def run_tdt():
        r = oracle.RnntOracle(hp, t)
        t0 = time.perf_counter()
        r.decode(enc)
        return time.perf_counter() - t0

    return {"frames": T, "tokens": len(got), "ms_per_decode": round(best * 1e3, 3),
            "decodes_per_s": round(1.0 / best, 1), "parity_bit_exact": bool(same),
            "cpu_baseline": {**vnni_baseline(run_tdt, 1.0, "decodes/s", "the same decode on the oracle"),
                             "scalar_one_thread": round(1.0 / cpu_s, 2)}}


def profile_leg(args) -> dict:
    """One workload alone, as the committed profiles run it."""
    leg = args.profile_leg
    if leg == "speak":
        # the pocket flow LM (d 1024, 6 layers) with the flow head (512, 6
        # residual blocks, 1 LSD step): a 64-row prefix, then 40 frames
        from gorelaxor_amd.pocket import PocketLM
        from gorelaxor_amd.synth import POCKET_FLOW, POCKET_TTS_LM, pocket_flow_model, pocket_inputs, pocket_model
        hp, fhp = dict(POCKET_TTS_LM), dict(POCKET_FLOW)
        t, ft = pocket_model(hp, seed=5), pocket_flow_model(hp, fhp, seed=7)
        x, _ = pocket_inputs(hp, 1, prefix=64, seed=6)
        noise = np.random.default_rng(8).standard_normal((40, hp["ldim"])).astype(np.float32)
        lm = PocketLM(hp, t)
        lm.flow_init(fhp["dim"], fhp["depth"], fhp["steps"])
        for k, v in ft.items():
            lm.set_tensor(k, v)
        for _ in range(3):
            lm.reset()
            lm.run(x)
            t0 = time.perf_counter()
            lm.speak(noise)
            ms = (time.perf_counter() - t0) * 1e3
        lm.close()
        return {"leg": leg, "frames": 40, "ms_last_speak": round(ms, 3)}
    if leg == "tdt":
        # the Parakeet-TDT-shaped head over 125 frames of N(0, 1), 6 decodes
        from gorelaxor_amd.rnnt import TransducerDecoder
        from gorelaxor_amd.synth import RNNT_TDT, rnnt_encoder_output, rnnt_model
        hp = dict(RNNT_TDT)
        dec = TransducerDecoder(hp, rnnt_model(hp, seed=30))
        enc = rnnt_encoder_output(hp, 125, seed=31)
        for _ in range(6):
            toks = dec.decode(enc)
        dec.close()
        return {"leg": leg, "frames": 125, "tokens": len(toks)}
    if leg == "sampler":
        # whisper's rules and sampler over 51,864 logits (one text token,
        # temperature 0): 21 calls for each of three logit kinds
        from gorelaxor_amd.whisper import Rules, sample_logits, special_tokens
        n = 51864
        sp = special_tokens(n)
        rules = Rules(sp, [1, 2, 7, 8, 9, 10, 220, 1906, 3556, 50254], space=220)
        rng = np.random.default_rng(3)
        beg = sp["beg"]
        kinds = {"wide": (rng.standard_normal(n) * 6.0).astype(np.float32)}
        lg = (rng.standard_normal(n) * 2.5).astype(np.float32)
        lg[rng.integers(0, beg, 5)] += 18.0
        lg[beg:] -= 6.0
        kinds["spread"] = lg
        kinds["flat"] = (rng.standard_normal(n) * 0.05).astype(np.float32)
        out = {}
        for name, lg in kinds.items():
            for _ in range(21):
                tok = sample_logits(lg, rules, tokens=[300])
            out[name] = tok["id"]
        return {"leg": leg, "ids": out}
    if leg == "mimi":
        # the Mimi decoder at the english_2026-09 shape, 40 latents one per
        # call, after 8 to warm up
        from gorelaxor_amd.mimi import MimiDecoder
        from gorelaxor_amd.synth import MIMI, mimi_latents, mimi_model
        hp = dict(MIMI)
        dec = MimiDecoder(hp, mimi_model(hp, seed=17), max_latents=1)
        lat = mimi_latents(hp, 48, seed=18)
        for k in range(48):
            dec.decode(lat[k:k + 1])
        dec.close()
        return {"leg": leg, "latents": 48}
    # the streaming chunk steps alone
    return {"leg": leg, "conformer_stream": conformer_stream_bench(args)}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus must be 1",
                          "detail": "the path shards data-parallel by stream/utterance with no exchange"}))
        sys.exit(2)

    from gorelaxor_amd import hiprt, kern

    if args.profile_leg:
        print(json.dumps(profile_leg(args)), flush=True)
        return
    if args.copy_calibration:
        nbytes = N * RING * K // 32 * 34
        a, b = hiprt.DeviceBuffer(nbytes), hiprt.DeviceBuffer(nbytes)
        a.zero()
        for _ in range(3):
            b.copy_from(a)
        hiprt.synchronize()
        print(json.dumps({"copy_calibration_bytes": nbytes, "copies": 3}), flush=True)
        return

    ctx = kern.default_context(0)
    stream = ctx.stream
    w8, x = ring_weights()
    w = kern.NewQ8(N * RING, K, w8, ctx)
    dx = hiprt.DeviceBuffer.from_array(x)
    dy = hiprt.DeviceBuffer(N * RING * 4)
    hiprt.synchronize()

    # one step = one launch: the product rounds x to Q8_0 in its prologue
    def step(evs=None, i=0):
        if evs is not None:
            evs[0][i].record(stream)
        kern.matmul_dev(dy, dx, 1, w, ctx=ctx)
        if evs is not None:
            evs[1][i].record(stream)

    for _ in range(args.warmup):
        step()
    ctx.sync()

    # the timed region: `steps` launches back to back, bracketed by events
    start, end = hiprt.Event(), hiprt.Event()
    ctx.sync()
    start.record(stream)
    t0 = time.perf_counter()
    for i in range(args.steps):
        step()
    end.record(stream)
    ctx.sync()
    wall = time.perf_counter() - t0
    total_ms = start.elapsed_ms(end)
    ms_step = total_ms / args.steps
    # the kernel's own duration: the same steps again, each launch between
    # its own pair of events on the library's stream (an event record
    # between launches adds a few us of gap, so it stays out of the timed
    # region above)
    ev = [[hiprt.Event() for _ in range(args.steps)] for _ in range(2)]
    for i in range(args.steps):
        step(ev, i)
    ctx.sync()
    gemv_ms = [ev[0][i].elapsed_ms(ev[1][i]) for i in range(args.steps)]
    gemv_avg = float(np.mean(gemv_ms))
    launch_bytes = BYTES_PER_GEMV * RING
    value = launch_bytes / (ms_step * 1e-3) / 1e9
    achieved = launch_bytes / (gemv_avg * 1e-3) / 1e9

    # one 1024 x 1024 matrix on its own (the reference's kernel-benchmark
    # shape): launches back to back, and each launch waited for
    w1 = kern.NewQ8(N, K, w8[:N * K // 32 * 34], ctx)
    dy1 = hiprt.DeviceBuffer(N * 4)
    for _ in range(20):
        kern.matmul_dev(dy1, dx, 1, w1, ctx=ctx)
    ctx.sync()
    a1, b1 = hiprt.Event(), hiprt.Event()
    a1.record(stream)
    for _ in range(200):
        kern.matmul_dev(dy1, dx, 1, w1, ctx=ctx)
    b1.record(stream)
    ctx.sync()
    single_us = a1.elapsed_ms(b1) / 200 * 1e3
    t0 = time.perf_counter()
    for _ in range(200):
        kern.matmul_dev(dy1, dx, 1, w1, ctx=ctx)
        ctx.sync()
    single_sync_us = (time.perf_counter() - t0) / 200 * 1e6
    del w1, dy1

    # parity spot check of this very run against the oracle (first matrix)
    import oracle
    oracle.build()
    want = oracle.matmul_q8_int(x, w8[:N * K // 32 * 34], N, K)[0]
    got = dy.download(np.float32, (N,))
    parity = bool(np.array_equal(got.view(np.uint32), want.view(np.uint32)))

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "q8_0 GEMV 1024x1024 over a ring of 512 distinct matrices (570 MB) per step, "
                               "x rounded to Q8_0 on the fly", "n": N, "k": K, "ring": RING,
                   "bytes_per_step": launch_bytes, "hbm_fraction": round(value / HBM_PEAK_GBS, 4),
                   "parity_bit_exact": parity, "wall_s": round(wall, 3),
                   "single_matrix": {"us_per_gemv_back_to_back": round(single_us, 2),
                                     "us_per_gemv_synchronized": round(single_sync_us, 2),
                                     "gbs_back_to_back": round(BYTES_PER_GEMV / (single_us * 1e-6) / 1e9, 1)}},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "kernel": "gemv1_kernel<1,4,QUANT,STORE>", "kernel_avg_us": round(gemv_avg * 1e3, 3)},
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(w8, x, args.cpu_seconds)
    del w, dy, dx
    if not args.no_decoder:
        out["decoder"] = decoder_bench(args)
        out["config"]["workload"] += "; whisper base.en-shaped greedy decoder (decoder.tokens_per_s)"
    if not args.no_streams:
        out["streams"] = streams_bench(args)
        out["config"]["workload"] += "; large-v3-turbo-shaped decoder, 8 streams batched (streams.tokens_per_s)"
    if not args.no_lm:
        out["lm"] = lm_bench(args)
        out["config"]["workload"] += "; pocket-TTS-style flow-LM frame loop (lm.frames_per_s)"
    if not args.no_conformer:
        out["conformer"] = conformer_bench(args)
        out["config"]["workload"] += "; parakeet-shaped conformer encoder at batch 1 and 16 (conformer.*)"
    if not args.no_conformer_stream:
        out["conformer_stream"] = conformer_stream_bench(args)
        out["config"]["workload"] += ("; Nemotron-streaming-shaped chunk steps at right contexts 13 and 0, "
                                      "1 and 16 streams (conformer_stream.*)")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
