"""The reference's float16 whisper decode on the CPU (the timing context of
the decoder benchmark): it runs the decoder.go graph with float16 matrices.
Its logits are close to the Q8_0 oracle's (the same model, matrices rounded
to float16 instead of kept as Q8_0 blocks) and its incremental decode
equals its prompt decode within float32 noise."""
import numpy as np
import pytest

import oracle
from gorelaxor_amd.synth import WHISPER_TINY_TEST, encoder_output, whisper_model


@pytest.mark.parametrize("threads", [1, 4])
def test_f16_decode_tracks_q8_oracle(threads):
    hp = dict(WHISPER_TINY_TEST)
    t = whisper_model(hp, seed=5)
    ref = oracle.WhisperOracle(hp, t)
    ref.set_encoder_output(encoder_output(hp, seed=6))
    f16 = oracle.WhisperF16(ref, t)
    toks = [5, 17, 3, 99]
    want = ref.decode(toks)
    got = f16.decode(toks, threads).copy()
    # float16 matrices vs Q8_0 blocks of the same weights: each weight
    # differs by at most half a float16 ulp, the logits by a few percent of
    # their spread
    spread = float(want.max() - want.min())
    assert np.abs(got - want).max() < 0.05 * spread
    assert np.corrcoef(got, want)[0, 1] > 0.999
    # one token at a time gives the prompt call's values (same kernels per row)
    f16.reset()
    for tok in toks:
        one = f16.decode([tok], threads).copy()
    np.testing.assert_allclose(one, got, rtol=1e-5, atol=1e-5 * spread)


def test_f16_decode_rejects_long_calls():
    hp = dict(WHISPER_TINY_TEST)
    t = whisper_model(hp, seed=5)
    ref = oracle.WhisperOracle(hp, t)
    ref.set_encoder_output(encoder_output(hp, seed=6))
    f16 = oracle.WhisperF16(ref, t)
    with pytest.raises(ValueError):
        f16.decode(list(range(6)))
