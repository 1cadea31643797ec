"""whisper's token rules and sampler on the GPU (grx_whisper_sample_logits,
grx_whisper_sample) against the oracle (session.process + session.sample,
whisper/transcribe.go:370-536): the sampled token, its best timestamp, the
timestamp rule's decision and the float32 bits of p and plog identical, over
logits whose sums keep few terms and logits where every term counts (several
LDS rounds of the left-to-right sum), every sequence state the rules read,
temperatures 0 to 1 and draws, English and multilingual vocabularies, and
on the logits a decode leaves on the device."""
import time

import numpy as np
import pytest

from gorelaxor_amd.whisper import Rules, special_tokens

pytestmark = pytest.mark.gpu

EN, ML = 51864, 51866
SUPPRESS = [1, 2, 7, 8, 9, 10, 220, 1906, 3556, 50254]


def _logits(kind, n, sp, seed):
    rng = np.random.default_rng(seed)
    beg = sp["beg"]
    if kind == "spread":  # confident: a few tokens far above the rest
        lg = (rng.standard_normal(n) * 2.5).astype(np.float32)
        lg[rng.integers(0, beg, 5)] += 18.0
        lg[beg:] -= 6.0
    elif kind == "flat":  # every term of every sum counts
        lg = (rng.standard_normal(n) * 0.05).astype(np.float32)
    elif kind == "wide":
        lg = (rng.standard_normal(n) * 6.0).astype(np.float32)
    elif kind == "timestamps":  # the timestamps together outweigh the text
        lg = (rng.standard_normal(n) * 1.5 - 8.0).astype(np.float32)
        lg[beg:beg + 200] = (rng.standard_normal(200) * 0.5 + 1.0).astype(np.float32)
        lg[rng.integers(0, beg)] = 4.0
    elif kind == "ties":
        lg = np.full(n, -3.0, np.float32)
        lg[[777, 123, 4000]] = 6.0
        lg[beg + 10: beg + 13] = 2.0
    return lg


SEQS = {
    "initial": dict(tokens=[]),
    "text": dict(tokens=[100, 200]),
    "ts_open": dict(tokens=[100, "beg+12"]),
    "ts_pair": dict(tokens=["beg+11", "beg+12"], has_ts=True, seek_delta=24),
    "has_ts": dict(tokens=[100, 300], has_ts=True, seek_delta=40),
}


def _seq(name, sp):
    s = dict(SEQS[name])
    s["tokens"] = [sp["beg"] + int(t[4:]) if isinstance(t, str) else t for t in s["tokens"]]
    return s


def _same(got, want):
    return (got["id"], got["tid"], got["force_ts"]) == (want["id"], want["tid"], want["force_ts"]) and \
        np.float32(got["p"]).view(np.uint32) == np.float32(want["p"]).view(np.uint32) and \
        np.float32(got["plog"]).view(np.uint32) == np.float32(want["plog"]).view(np.uint32)


@pytest.mark.parametrize("n", [EN, ML])
@pytest.mark.parametrize("kind", ["spread", "flat", "wide", "timestamps", "ties"])
def test_sample_bit_exact(kern, orc, n, kind):
    from gorelaxor_amd.whisper import sample_logits

    sp = special_tokens(n)
    rules = Rules(sp, SUPPRESS, space=220)
    rng = np.random.default_rng(n + len(kind))
    for si, seq_name in enumerate(SEQS):
        lg = _logits(kind, n, sp, seed=si * 7 + len(kind))
        seq = _seq(seq_name, sp)
        for temp in (0.0, 0.2, 0.6, 1.0):
            r = float(np.float32(rng.random()))
            got = sample_logits(lg, rules, temp=temp, r=r, **seq)
            want = orc.whisper_sample(lg, sp, suppress=SUPPRESS, space=220, temp=temp, r=r, **seq)
            assert _same(got, want), (kind, seq_name, temp, r, got, want)


def test_sample_timestamp_rule_fires(kern, orc):
    """The timestamp logits are built to win: the rule forces a timestamp on
    the GPU as in the oracle."""
    from gorelaxor_amd.whisper import sample_logits

    sp = special_tokens(EN)
    lg = _logits("timestamps", EN, sp, seed=4)
    got = sample_logits(lg, Rules(sp, SUPPRESS), tokens=[100, 200])
    want = orc.whisper_sample(lg, sp, suppress=SUPPRESS, tokens=[100, 200])
    assert want["force_ts"] and _same(got, want)


def test_sample_on_decoder_logits(kern, orc):
    """After a decode, the rules and sampler read the logits where the step
    left them; the result is the oracle's on those logits."""
    from gorelaxor_amd.synth import encoder_output, whisper_model
    from gorelaxor_amd.whisper import WhisperDecoder, sample_logits

    hp = dict(n_vocab=EN, n_text_ctx=64, n_state=128, n_head=2, n_layer=2, n_audio_ctx=1500)
    dec = WhisperDecoder(hp, whisper_model(hp, seed=9))
    dec.set_encoder_output(encoder_output(hp, seed=10))
    sp = special_tokens(EN)
    rules = Rules(sp, SUPPRESS, space=220)
    lg, _ = dec.decode([sp["sot"], 300, 400])
    for temp, r in ((0.0, 0.0), (0.4, 0.37)):
        got = dec.sample(rules, tokens=[300], temp=temp, r=r)
        want = orc.whisper_sample(lg, sp, suppress=SUPPRESS, space=220, tokens=[300], temp=temp, r=r)
        assert _same(got, want), (temp, got, want)
    t0 = time.perf_counter()
    for _ in range(50):
        dec.sample(rules, tokens=[300])
    dt = (time.perf_counter() - t0) / 50
    t0 = time.perf_counter()
    for _ in range(20):
        sample_logits(lg, rules, tokens=[300])
    dt2 = (time.perf_counter() - t0) / 20
    print(f"\nsample on device logits: {dt * 1e6:.1f} us per call; from host logits: {dt2 * 1e6:.1f} us", flush=True)
    for kind in ("spread", "wide", "flat"):
        x = _logits(kind, EN, sp, seed=1)
        t0 = time.perf_counter()
        for _ in range(20):
            sample_logits(x, rules, tokens=[300])
        print(f"host logits, {kind}: {(time.perf_counter() - t0) / 20 * 1e6:.1f} us", flush=True)
    dec.close()


def test_sample_errors(kern):
    from gorelaxor_amd import GrxError
    from gorelaxor_amd.whisper import sample_logits

    sp = special_tokens(EN)
    with pytest.raises(GrxError, match="outside"):
        sample_logits(np.zeros(1000, np.float32), Rules(sp))
