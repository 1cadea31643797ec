"""The decode loop of one whisper window on the device (grx_whisper_rules_loop,
whisper/transcribe.go:207-260): each iteration's token rules and sampler
(process + sample, transcribe.go:370-494) with the sequence state held in
device memory, the loop's timestamp, end and stuck rules, and the token fed
to the next decode step without a host round trip.  Against the oracle's
restatement of the same loop (its decode and sampler): every token's id,
best timestamp, the timestamp rule's decision and the bits of p and plog,
and the sequence state the loop leaves, at temperature 0 and with draws."""
import numpy as np
import pytest

from gorelaxor_amd.synth import encoder_output, whisper_model
from gorelaxor_amd.whisper import Rules, special_tokens

pytestmark = pytest.mark.gpu

EN = 51864
SUPPRESS = [1, 2, 7, 8, 9, 10, 220, 1906, 3556, 50254]


def _same_tok(g, w):
    return (g["id"], g["tid"], g["force_ts"]) == (w["id"], w["tid"], w["force_ts"]) and \
        np.float32(g["p"]).view(np.uint32) == np.float32(w["p"]).view(np.uint32) and \
        np.float32(g["plog"]).view(np.uint32) == np.float32(w["plog"]).view(np.uint32)


def _scaled(t, hp, factor, ts_factor):
    """The token embedding's block scales times factor (timestamp rows times
    factor * ts_factor): flatter logits, so that draws and the timestamp
    rules come into play (the random-init model's logits are peaked enough
    to repeat one token)."""
    sp = special_tokens(hp["n_vocab"])
    w = np.asarray(t["decoder.token_embedding.weight"]).copy().reshape(hp["n_vocab"], hp["n_state"] // 32, 34)
    sc = np.ascontiguousarray(w[:, :, :2]).view(np.float16)[..., 0].astype(np.float32)
    f = np.full(hp["n_vocab"], factor, np.float32)
    f[sp["beg"]:] *= ts_factor
    w[:, :, :2] = (sc * f[:, None]).astype(np.float16)[..., None].view(np.uint8)
    t = dict(t)
    t["decoder.token_embedding.weight"] = w.reshape(-1)
    return t


def _pair(orc, hp, seed, factor=1.0, ts_factor=1.0):
    from gorelaxor_amd.whisper import WhisperDecoder

    t = whisper_model(hp, seed=seed)
    if factor != 1.0 or ts_factor != 1.0:
        t = _scaled(t, hp, factor, ts_factor)
    enc = encoder_output(hp, seed=seed + 1)
    ref = orc.WhisperOracle(hp, t)
    ref.set_encoder_output(enc)
    dec = WhisperDecoder(hp, t)
    dec.set_encoder_output(enc)
    return ref, dec


CASES = {
    # n_text_ctx, prompt, seek, seek_end, temp, timestamps suppressed, embedding scale, timestamp rows' extra scale
    "greedy": (64, "sot", 0, 30000, 0.0, False, 1.0, 1.0),  # one token repeated: stuck, failed at the end
    "no_ts": (128, "sot", 0, 30000, 0.0, True, 1.0, 1.0),
    "ts_greedy": (128, "sot", 0, 30000, 0.0, False, 0.1, 6.0),  # timestamps win often: pairs, the forcing rule
    "draws": (128, "sot", 0, 30000, 1.0, False, 0.05, 1.0),
    "ts_draws": (128, "past", 3000, 30000, 0.7, False, 0.05, 4.0),
    "near_end": (128, "sot", 2000, 2800, 1.0, False, 0.05, 3.0),  # a timestamp reaches the audio's end: done
    "mixed": (128, "past", 0, 30000, 0.5, False, 0.1, 3.0),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_loop_bit_exact(kern, orc, case):
    ctxn, pk, seek, seek_end, temp, no_ts, factor, tsf = CASES[case]
    hp = dict(n_vocab=EN, n_text_ctx=ctxn, n_state=128, n_head=2, n_layer=2, n_audio_ctx=1500)
    sp = special_tokens(EN)
    sup = SUPPRESS + (list(range(sp["beg"], EN)) if no_ts else [])
    rules = Rules(sp, sup, space=220)
    ref, dec = _pair(orc, hp, seed=3 + len(case), factor=factor, ts_factor=tsf)
    prompt = [sp["sot"]] if pk == "sot" else [sp["prev"], 400, 13, 77, sp["sot"]]
    n_max = ctxn // 2 - 4
    rng = np.random.default_rng(len(case))
    draws = rng.random(n_max).astype(np.float32)
    lr = ref.decode(prompt)
    lg, _ = dec.decode(prompt)
    want, wst = orc.whisper_window_loop(ref, lr, sp, suppress=sup, space=220, seek=seek, seek_end=seek_end,
                                        n_max=n_max, temp=temp, r=draws)
    got, gst = dec.rules_loop(rules, seek, seek_end, n_max, temp=temp, r=draws)
    assert gst == wst, (gst, wst)
    assert len(got) == len(want)
    for k, (g, w) in enumerate(zip(got, want)):
        assert _same_tok(g, w), (k, g, w)
    print(f"\n{case}: {wst}, {sum(w['id'] >= sp['beg'] for w in want)} timestamps, "
          f"{sum(w['force_ts'] for w in want)} forced", flush=True)


def test_loop_errors(kern, orc):
    from gorelaxor_amd import GrxError
    from gorelaxor_amd.whisper import WhisperDecoder

    hp = dict(n_vocab=EN, n_text_ctx=64, n_state=128, n_head=2, n_layer=2, n_audio_ctx=1500)
    sp = special_tokens(EN)
    rules = Rules(sp, SUPPRESS, space=220)
    ref, dec = _pair(orc, hp, seed=2)
    with pytest.raises(GrxError, match="no prompt"):
        dec.rules_loop(rules, 0, 3000, 10)
    dec.decode([sp["sot"]])
    with pytest.raises(GrxError, match="exceed the context"):
        dec.rules_loop(rules, 0, 3000, 64)
    two = WhisperDecoder(hp, whisper_model(hp, seed=2), streams=2)
    two.set_encoder_output_stream(0, encoder_output(hp, seed=3))
    two.share_encoder_output(1, 0)
    with pytest.raises(GrxError, match="streams"):
        two.rules_loop(rules, 0, 3000, 4)
