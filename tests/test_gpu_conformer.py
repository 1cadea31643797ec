"""GPU parity of the FastConformer encoder (conformer/encoder.go:432-489)
against the CPU oracle: bit-identical outputs for every utterance of a
batch, at a tiny shape (both convolution norms, Q8_0 and float16 pointwise
weights), at the full parakeet width with two layers, and at all 24
layers for the 10 s input, with batching shown not to change an
utterance's output."""
import numpy as np
import pytest

from gorelaxor_amd.synth import CONFORMER_TINY, PARAKEET_TDT_06B, conformer_model, noise_mel

pytestmark = pytest.mark.gpu


def _enc(kern, hp, t):
    from gorelaxor_amd.conformer import ConformerEncoder
    return ConformerEncoder(hp, t)


def _mels(hp, n, seconds, seed):
    out = [noise_mel(hp["n_mels"], seconds=seconds, seed=seed + i) for i in range(n)]
    return np.stack([m for m, _, _ in out]), out[0][1], out[0][2]


@pytest.mark.parametrize("conv_norm,f16", [("batch_norm", True), ("batch_norm", False), ("layer_norm", True)])
def test_tiny_encode_bit_exact(kern, orc, conv_norm, f16):
    hp = dict(CONFORMER_TINY, conv_norm=conv_norm)
    t = conformer_model(hp, seed=21, pointwise_f16=f16)
    mel, frames, valid = _mels(hp, 3, 1.5, 30)
    vals = [valid, valid - 9, valid - 40]
    enc = _enc(kern, hp, t)
    got, lens = enc.encode(mel, vals)
    o = orc.ConformerOracle(hp, t)
    for b in range(3):
        want, L = o.encode(mel[b], vals[b])
        assert lens[b] == L
        assert np.array_equal(got[b].view(np.uint32), want.view(np.uint32)), (b, np.abs(got[b] - want).max())
    enc.close()


@pytest.mark.parametrize("seconds", [1.5, 0.07])
def test_tiny_float32_pre_encoder_pointwise(kern, orc, seconds):
    """conv.3 and conv.6 stored float32, as the reference's converter writes
    them: kern.Linear's float route (rows in whole groups of six by the
    k6x16 chain, the rest by gemvRows; at 0.07 s every row takes gemvRows),
    bit-identical to the oracle."""
    hp = dict(CONFORMER_TINY)
    t = conformer_model(hp, seed=25, pre_f32=True)
    assert t["enc.pre_encode.conv.3.weight"].dtype == np.float32
    mel, frames, valid = _mels(hp, 2, seconds, 36)
    vals = [valid, max(1, valid - 3)]
    enc = _enc(kern, hp, t)
    got, lens = enc.encode(mel, vals)
    o = orc.ConformerOracle(hp, t)
    for b in range(2):
        want, L = o.encode(mel[b], vals[b])
        assert lens[b] == L
        assert np.array_equal(got[b].view(np.uint32), want.view(np.uint32)), (b, np.abs(got[b] - want).max())
    enc.close()


@pytest.mark.parametrize("rq", [0, 4, 8, 16])
def test_tiny_attention_variants_bit_exact(kern, orc, rq):
    """The unstaged attention kernel and the LDS-staged one at 8 and 16 query
    rows per workgroup give the same bits as the oracle (T = 19: one query
    block, rows in the 6x16 panels and in gemvRows)."""
    hp = dict(CONFORMER_TINY)
    t = conformer_model(hp, seed=24)
    mel, frames, valid = _mels(hp, 2, 1.5, 35)
    vals = [valid, valid - 30]
    with kern.tuned(CONF_ATTN_RQ=rq):
        enc = _enc(kern, hp, t)
        got, lens = enc.encode(mel, vals)
    o = orc.ConformerOracle(hp, t)
    for b in range(2):
        want, L = o.encode(mel[b], vals[b])
        assert np.array_equal(got[b].view(np.uint32), want.view(np.uint32)), (rq, b)
    enc.close()


@pytest.mark.parametrize("dw", [0, 1, 2])
def test_depthwise_variants_bit_exact(kern, orc, dw):
    """Every depthwise kernel - a workgroup per row, LDS windows, a wave per
    frame - gives the oracle's bits: the tiny shape (kernel 9) with
    utterances whose padding rows the GLU zeroes, and the parakeet width
    (kernel 31) with two layers."""
    hp = dict(CONFORMER_TINY)
    t = conformer_model(hp, seed=26)
    mel, frames, valid = _mels(hp, 3, 1.5, 37)
    vals = [valid, valid - 9, valid - 60]
    with kern.tuned(CONF_DW=dw):
        enc = _enc(kern, hp, t)
        got, lens = enc.encode(mel, vals)
        enc.close()
    o = orc.ConformerOracle(hp, t)
    for b in range(3):
        want, L = o.encode(mel[b], vals[b])
        assert np.array_equal(got[b].view(np.uint32), want.view(np.uint32)), (dw, b)
    hp = dict(PARAKEET_TDT_06B, layers=2)
    t = conformer_model(hp, seed=33)
    mel, frames, valid = _mels(hp, 2, 10.0, 61)
    with kern.tuned(CONF_DW=dw):
        enc = _enc(kern, hp, t)
        got, lens = enc.encode(mel, [valid, valid - 250])
        enc.close()
    o = orc.ConformerOracle(hp, t)
    for b, v in enumerate([valid, valid - 250]):
        want, L = o.encode(mel[b], v)
        assert np.array_equal(got[b].view(np.uint32), want.view(np.uint32)), (dw, b)


@pytest.mark.parametrize("fuse,gk", [(0, -1), (1, -1), (3, -1), (1, 3)])
def test_tiny_fused_layernorms(kern, orc, fuse, gk):
    """One utterance of 0.7 s (9 rows: one 16-row group), two of 0.5 s and
    three of 0.7 s (27 rows: a second, partial group): with CONF_FUSE=3 the
    K-split products take the blocks' LayerNorms in their prologues (a
    block's norm_out and the next one's LayerNorm in the first); by default
    pointwise1 takes its GLU; with CONF_FUSE=0 each is a launch of its own;
    on the LDS tiles (GEMM_KERNEL=3) pointwise1 takes the GLU there - every
    form bit-identical to the oracle."""
    hp = dict(CONFORMER_TINY, layers=3)
    t = conformer_model(hp, seed=27)
    o = orc.ConformerOracle(hp, t)
    with kern.tuned(CONF_FUSE=fuse, GEMM_KERNEL=gk):
        enc = _enc(kern, hp, t)
        for seconds, n in ((0.7, 1), (0.5, 2), (0.7, 3)):
            mel, frames, valid = _mels(hp, n, seconds, 41)
            lens_in = [valid, valid - 7, valid - 3][:n]
            print(f"fused layernorms fuse {fuse} gk {gk}: {n} x {seconds} s", flush=True)
            got, lens = enc.encode(mel, lens_in)
            for b in range(n):
                want, L = o.encode(mel[b], lens_in[b])
                assert np.array_equal(got[b].view(np.uint32), want.view(np.uint32)), (fuse, seconds, b)
        enc.close()


def test_tiny_shape_change_and_rerun(kern, orc):
    """A second call with another batch and frame count re-plans the work;
    repeating a call gives the same bits."""
    hp = dict(CONFORMER_TINY)
    t = conformer_model(hp, seed=22)
    enc = _enc(kern, hp, t)
    o = orc.ConformerOracle(hp, t)
    for seconds, n in ((1.0, 2), (0.7, 1), (1.0, 2)):
        mel, frames, valid = _mels(hp, n, seconds, 40)
        got, lens = enc.encode(mel, valid)
        for b in range(n):
            want, L = o.encode(mel[b], valid)
            assert np.array_equal(got[b].view(np.uint32), want.view(np.uint32)), (seconds, b)
    enc.close()


def test_bad_input_errors(kern):
    from gorelaxor_amd._lib import GrxError
    hp = dict(CONFORMER_TINY)
    t = conformer_model(hp, seed=23)
    enc = _enc(kern, hp, None)
    with pytest.raises(GrxError, match="EINVAL"):
        enc.set_tensor("enc.blocks.0.no_such.weight", np.zeros(4, np.float32))
    with pytest.raises(GrxError, match="ESIZE"):
        enc.set_tensor("enc.blocks.0.norm_out.weight", np.zeros(3, np.float32))
    mel, frames, valid = _mels(hp, 1, 1.0, 50)
    with pytest.raises(GrxError, match="ESTATE"):
        enc.encode(mel, valid)  # no tensors yet
    for k, v in t.items():
        enc.set_tensor(k, v)
    with pytest.raises(GrxError, match="EINVAL"):
        enc.encode(mel, frames + 1)
    enc.close()


@pytest.fixture(scope="module", params=[False, True], ids=["q8_pre", "f32_pre"])
def parakeet2(request):
    hp = dict(PARAKEET_TDT_06B, layers=2)
    return hp, conformer_model(hp, seed=31, pre_f32=request.param)


def test_parakeet_width_two_layers_bit_exact(kern, orc, parakeet2):
    """10 s of noise, d 1024, 8 heads, FFN 4096, kernel 31, 128 mels: the
    pre-encoder (its conv.3 and conv.6 Q8_0, or float32 as converted files
    hold them) and two blocks bit-identical to the oracle."""
    hp, t = parakeet2
    mel, frames, valid = _mels(hp, 1, 10.0, 60)
    enc = _enc(kern, hp, t)
    got, lens = enc.encode(mel, valid)
    want, L = orc.ConformerOracle(hp, t).encode(mel[0], valid)
    assert (got.shape[1], lens[0], L) == (126, 125, 125)
    assert np.array_equal(got[0].view(np.uint32), want.view(np.uint32)), np.abs(got[0] - want).max()
    enc.close()


def test_parakeet_24_layers_bit_exact_and_batched(kern, orc):
    """All 24 layers at batch 4 (utterances of different valid lengths): the
    first (the full 10 s) bit-identical to the oracle, and a shorter one
    equal to its own batch-1 encode, bit for bit."""
    hp = dict(PARAKEET_TDT_06B)
    t = conformer_model(hp, seed=32)
    mel, frames, valid = _mels(hp, 4, 10.0, 70)
    vals = [valid, valid - 100, valid - 333, valid]
    enc = _enc(kern, hp, t)
    got, lens = enc.encode(mel, vals)
    assert list(lens) == [125, 113, 84, 125]
    one, l1 = enc.encode(mel[2:3], vals[2])
    assert np.array_equal(one[0].view(np.uint32), got[2].view(np.uint32))
    enc.close()
    want, L = orc.ConformerOracle(hp, t).encode(mel[0], vals[0])
    assert L == 125
    assert np.array_equal(got[0].view(np.uint32), want.view(np.uint32)), np.abs(got[0] - want).max()
    x = got[0, :125]
    assert np.isfinite(x).all() and 0.3 < float(np.abs(x).mean()) < 3.0


def test_parakeet_24_layers_batch16(kern, orc):
    """The configuration's batch of 16: sixteen 10 s noise utterances through
    all 24 layers at once (the batch whose attention takes the 16-query-row
    LDS kernel at T = 126).  Each utterance's output is bit-identical to its
    own batch-1 encode, and utterance 0 to the oracle."""
    hp = dict(PARAKEET_TDT_06B)
    t = conformer_model(hp, seed=32)
    mel, frames, valid = _mels(hp, 16, 10.0, 70)
    enc = _enc(kern, hp, t)
    got, lens = enc.encode(mel, valid)
    assert got.shape[:2] == (16, 126) and list(lens) == [125] * 16
    for i in range(16):
        one, _ = enc.encode(mel[i:i + 1], valid)
        assert np.array_equal(one[0].view(np.uint32), got[i].view(np.uint32)), i
    enc.close()
    want, L = orc.ConformerOracle(hp, t).encode(mel[0], valid)
    assert L == 125
    assert np.array_equal(got[0].view(np.uint32), want.view(np.uint32)), np.abs(got[0] - want).max()
