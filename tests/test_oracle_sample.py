"""The oracle of whisper's token rules and sampler (session.process and
session.sample, whisper/transcribe.go:370-536) pinned by what the rules and
the mathematics fix: each suppression rule on logits that would otherwise
pick the suppressed token, the timestamp rule on both sides of its
threshold, log probabilities and probabilities against float64 closed
forms, the draw's cumulative bracket, the temperature's scaling, and the
special token table of newVocab (whisper/vocab.go:20-45)."""
import math

import numpy as np
import pytest

from gorelaxor_amd.whisper import special_tokens

EN, ML = 51864, 51866


def test_special_tokens_table():
    """vocab.go:28-45: English ids; a v3 (51866) vocabulary: 100 languages,
    eot/sot one later, the task and timestamp ids 2 later."""
    e = special_tokens(EN)
    assert (e["eot"], e["sot"], e["beg"], e["n_lang"]) == (50256, 50257, 50363, 0)
    m = special_tokens(ML)
    assert (m["eot"], m["sot"], m["translate"], m["no_timestamps"], m["beg"], m["n_lang"]) == \
        (50257, 50258, 50359, 50364, 50365, 100)
    assert special_tokens(51865)["beg"] == 50364 and special_tokens(51865)["n_lang"] == 99


def _flat(n, base=0.0):
    return np.full(n, base, np.float32)


def _go(orc, lg, sp, **kw):
    return orc.whisper_sample(lg, sp, **kw)


@pytest.mark.parametrize("rule", ["special", "language", "suppress", "initial_eot", "initial_space",
                                  "initial_ts_limit", "pair_done", "pair_open", "seek_delta"])
def test_each_rule_blocks_its_token(orc, rule):
    """A token the rule removes is made the largest logit; the sample must
    not be it (and is the next best), and without the rule's condition it
    is."""
    sp = special_tokens(ML)
    n, beg = ML, sp["beg"]
    lg = _flat(n, -30.0)  # low enough that the timestamps together never decide
    lg[100] = 5.0  # the runner-up, a text token
    kw, free = {}, {}
    if rule == "special":
        bad = sp["transcribe"]
    elif rule == "language":
        bad = sp["sot"] + 1 + 37
    elif rule == "suppress":
        bad = 220
        kw, free = dict(suppress=[7, 220, 9]), dict(suppress=[7, 9])
    elif rule == "initial_eot":
        bad = sp["eot"]
        kw, free = dict(tokens=[]), dict(tokens=[100])
    elif rule == "initial_space":
        bad = 220
        kw, free = dict(space=220, tokens=[]), dict(space=220, tokens=[100])
    elif rule == "initial_ts_limit":  # 1 s at 1500 audio positions: tid0 = 50
        bad = beg + 51
        kw, free = dict(tokens=[]), dict(tokens=[100])
    elif rule == "pair_done":  # two timestamps in a row: no third
        bad = beg + 7
        kw, free = dict(tokens=[beg + 3, beg + 4]), dict(tokens=[100, 101])
    elif rule == "pair_open":  # a timestamp after text: text must not follow (below eot)
        bad = 100
        lg[sp["eot"]] = 5.0  # eot and timestamps stay allowed
        lg[bad] = 9.0
        kw, free = dict(tokens=[200, beg + 3]), dict(tokens=[beg + 2, beg + 3])
    elif rule == "seek_delta":  # timestamps before the last one's
        bad = beg + 4
        kw, free = dict(tokens=[100], has_ts=True, seek_delta=10), dict(tokens=[100], has_ts=True, seek_delta=8)
    if rule != "pair_open":
        lg[bad] = 9.0
    got = _go(orc, lg, sp, **({"tokens": [100]} | kw))
    assert got["id"] != bad
    if rule == "pair_open":
        assert got["id"] == sp["eot"]
    else:
        assert got["id"] == 100
    if free:
        assert _go(orc, lg, sp, **free)["id"] == bad


def test_log_probs_and_probs_closed_form(orc):
    """Three live tokens (the rest suppressed by -inf logits): plog and p
    against float64 closed forms, to float32 rounding."""
    sp = special_tokens(EN)
    lg = np.full(EN, -np.inf, np.float32)
    lg[[10, 20, 30]] = [1.25, 3.0, -0.5]
    got = _go(orc, lg, sp, tokens=[5])
    z = np.log(sum(math.exp(v) for v in (1.25, 3.0, -0.5)))
    assert got["id"] == 20
    assert abs(got["plog"] - (3.0 - z)) < 2e-6
    assert abs(got["p"] - math.exp(3.0 - z)) < 2e-6
    assert not got["force_ts"]


def test_temperature_scales_logits(orc):
    """At temperature 0.5 the log probability is that of the doubled logits."""
    sp = special_tokens(EN)
    lg = np.full(EN, -np.inf, np.float32)
    lg[[10, 20]] = [1.0, 2.0]
    got = _go(orc, lg, sp, tokens=[5], temp=0.5, r=0.99)
    z = np.log(math.exp(2.0) + math.exp(4.0))
    assert got["id"] == 20 and abs(got["plog"] - (4.0 - z)) < 2e-6


@pytest.mark.parametrize("text_lead, forced", [(1.5, True), (3.0, False)])
def test_timestamp_rule_threshold(orc, text_lead, forced):
    """Ten timestamps at logit L beat one text token at L + 1.5 (10 > e^1.5)
    but not at L + 3 (e^3 > 10): only the first forces a timestamp."""
    sp = special_tokens(EN)
    beg = sp["beg"]
    lg = np.full(EN, -np.inf, np.float32)
    lg[beg + 20: beg + 30] = 2.0
    lg[300] = 2.0 + text_lead
    got = _go(orc, lg, sp, tokens=[5])
    assert got["force_ts"] == forced
    assert (got["id"] >= beg) == forced
    if forced:
        assert got["id"] == beg + 20 and abs(got["p"] - 0.1) < 1e-6 and got["tid"] == got["id"]


def test_draw_brackets_r(orc):
    """The drawn token is the one whose cumulative probability first
    exceeds r (float64 check away from the bracket edges); r = 0 takes the
    first live token."""
    sp = special_tokens(EN)
    rng = np.random.default_rng(3)
    lg = (rng.standard_normal(EN) * 2).astype(np.float32)
    lg[sp["beg"]:] = -30.0  # the timestamps together must not decide
    ref = _go(orc, lg, sp, tokens=[5], temp=1.0, r=0.0)
    assert ref["id"] == 0
    for r in (0.1, 0.5, 0.93):
        got = _go(orc, lg, sp, tokens=[5], temp=1.0, r=r)
        live = lg.astype(np.float64)
        mask = np.zeros(EN, bool)
        for k in ("no_timestamps", "sot", "nosp", "solm", "translate", "transcribe", "prev"):
            mask[sp[k]] = True
        e = np.where(mask, 0.0, np.exp(live - live[~mask].max()))
        c = np.cumsum(e / e.sum())
        i = got["id"]
        assert c[i - 1] - 1e-4 <= r < c[i] + 1e-4 if i > 0 else r < c[0] + 1e-4


def test_argmax_ties_take_the_first(orc):
    sp = special_tokens(EN)
    lg = _flat(EN, -5.0)
    lg[[40, 30, 50]] = 3.0
    assert _go(orc, lg, sp, tokens=[5])["id"] == 30
