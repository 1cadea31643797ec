"""Pins the oracle's restatement of one window's decode loop
(whisper/transcribe.go:207-260, oracle.whisper_window_loop) without a GPU:
logits crafted so that the sampler must pick a chosen token at each
iteration, then every rule of the loop checked against its closed form -
a timestamp sets seekDelta = 2 (id - beg) and the result length; a
timestamp that goes back fails the sequence; eot finishes it, or fails it
when no result was kept and the audio has not ended; a timestamp reaching
the audio's end finishes it; the last iteration fails a sequence stuck
repeating itself; the loop decodes each token while the sequence runs."""
import numpy as np
import pytest

from gorelaxor_amd.whisper import special_tokens

EN = 51864
SP = special_tokens(EN)
BEG, EOT = SP["beg"], SP["eot"]


class Scripted:
    """Stands in for the decoder: the logits after each decoded token make
    the next scripted token the only likely one."""

    def __init__(self, script):
        self.script, self.fed = list(script), []

    def logits(self, k):
        lg = np.full(EN, -20.0, np.float32)
        lg[self.script[k]] = 30.0
        return lg

    def decode(self, toks):
        self.fed += list(toks)
        return self.logits(len(self.fed))


def _run(orc, script, **kw):
    ref = Scripted(script)
    toks, st = orc.whisper_window_loop(ref, ref.logits(0), SP, **kw)
    return [t["id"] for t in toks], st, ref.fed


def test_text_then_eot_without_timestamps_fails(orc):
    """eot with no result kept and the audio not at its end: failed."""
    ids, st, fed = _run(orc, [300, 301, EOT, 5], seek_end=30000, n_max=10)
    assert ids == [300, 301, EOT]
    assert st["failed"] == 1 and st["done"] == 0 and st["result_len"] == 0
    assert fed == [300, 301]  # no decode after the last sample


def test_timestamps_then_eot_done(orc):
    """A timestamp beg+k after text: seekDelta 2k, result length i+1; eot
    then finishes the sequence."""
    ids, st, _ = _run(orc, [300, BEG + 40, BEG + 41, 302, EOT], seek_end=30000, n_max=20)
    assert ids == [300, BEG + 40, BEG + 41, 302, EOT]
    assert st["done"] == 1 and st["failed"] == 0
    assert st["seek_delta"] == 82 and st["result_len"] == 3 and st["has_ts"] == 1


def test_timestamp_going_back_is_never_sampled(orc):
    """After timestamps up to beg+41 the rules take away beg..beg+40
    (transcribe.go:417-421), so a scripted beg+10 cannot be sampled: the
    sequence stays valid (the loop's going-back failure, :215-218, guards
    what the rules already prevent)."""
    script = [300, BEG + 40, BEG + 41, 302, 303, BEG + 10] + [400 + k for k in range(20)]
    ids, st, _ = _run(orc, script, seek_end=30000, n_max=8)
    assert ids[:5] == [300, BEG + 40, BEG + 41, 302, 303]
    assert ids[5] != BEG + 10 and not (BEG <= ids[5] < BEG + 41)
    # the last iteration: seekDelta 82 is under half a window, so it fails
    assert st["failed"] == 1 and st["seek_delta"] == 82
    assert len(ids) == 8


def test_timestamp_at_the_audio_end_done(orc):
    """seek + seekDelta + deltaMin >= seekEnd after a timestamp: done."""
    ids, st, _ = _run(orc, [300, BEG + 40, 5], seek=1000, seek_end=1085, n_max=20)
    assert ids == [300, BEG + 40] and st["done"] == 1 and st["result_len"] == 2


def test_eot_at_the_audio_end_keeps_its_length(orc):
    """eot with no timestamp but the window reaching the audio's end: the
    result is everything so far (result length i+1), done."""
    ids, st, _ = _run(orc, [300, 301, EOT], seek=0, seek_end=2500, n_max=20)
    assert st["done"] == 1 and st["result_len"] == 3


def test_stuck_at_the_last_iteration_fails(orc):
    """Text to the last iteration with no timestamp: failed there."""
    ids, st, fed = _run(orc, [300 + k for k in range(8)], seek_end=30000, n_max=6)
    assert len(ids) == 6 and st["failed"] == 1 and st["done"] == 0
    assert len(fed) == 5
