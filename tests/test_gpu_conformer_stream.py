"""GPU parity of cache-aware streaming (conformer/stream.go:23-88,
241-307) and of the limited-context offline encoder (conformer/encoder.go:
196-212, 343-404) against the CPU oracle, bit for bit:

  - offline encodes of a chunked-limited (causal) model and of a windowed
    one, every utterance of a batch;
  - streams chunk by chunk at right contexts 13, 6, 1 and 0, long enough
    for the key and convolution rings to wrap, with each chunk's rows equal
    to the oracle's streamStep; several streams stepped together, each
    equal to its own single-stream run; short last chunks and fewer real
    frames than the chunk holds;
  - the Nemotron-streaming shape (d 1024, 24 layers) at right contexts 13
    and 0: the M=14 and M=1 chunk steps;
  - the reference's errors: a model that can't stream, an untrained right
    context, a chunk with more rows than the geometry.
"""
import numpy as np
import pytest

from gorelaxor_amd import GrxError
from gorelaxor_amd.conformer import ConformerEncoder, ConformerStream, mel_chunks, stream_geom
from gorelaxor_amd.synth import CONFORMER_TINY, NEMOTRON_STREAMING, conformer_model, noise_mel

pytestmark = pytest.mark.gpu

STREAM_TINY = dict(CONFORMER_TINY, att_style="chunked_limited", att_left=70, att_right=13,
                   context_choices=[(70, 13), (70, 6), (70, 1), (70, 0)], conv_left=8, conv_right=0,
                   conv_norm="layer_norm")
# a shorter left context: the rings wrap within a few seconds
STREAM_TINY28 = dict(STREAM_TINY, att_left=28, context_choices=[(28, 13), (28, 6), (28, 1), (28, 0)])


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _same(got, want, what):
    assert got.shape == want.shape, (what, got.shape, want.shape)
    assert np.array_equal(_bits(got), _bits(want)), (what, float(np.abs(got - want).max()))


@pytest.mark.parametrize("hp", [STREAM_TINY, dict(CONFORMER_TINY, att_left=9, att_right=4)],
                         ids=["chunked", "window"])
def test_offline_limited_context_bit_exact(kern, orc, hp):
    t = conformer_model(hp, seed=31, pointwise_f16=True)
    mels = [noise_mel(hp["n_mels"], seconds=2.5, seed=50 + i) for i in range(3)]
    mel = np.stack([m for m, _, _ in mels])
    frames, valid = mels[0][1], mels[0][2]
    vals = [frames, valid - 5, valid - 60]
    enc = ConformerEncoder(hp, t)
    got, lens = enc.encode(mel, vals)
    o = orc.ConformerOracle(hp, t)
    for b in range(3):
        print(f"offline {hp.get('att_style', 'regular')} utterance {b}", flush=True)
        want, L = o.encode(mel[b], vals[b])
        assert lens[b] == L
        _same(got[b], want, b)
    enc.close()


def _stream_case(kern, orc, hp, t, right, seconds, seed, f16_note=""):
    mel, frames, _ = noise_mel(hp["n_mels"], seconds=seconds, seed=seed)
    enc = ConformerEncoder(hp, t)
    s = ConformerStream(enc, right)
    g = stream_geom(hp, right)
    assert {k: s.geom[k] for k in g if k != "sub"} == {k: v for k, v in g.items() if k != "sub"}
    o = orc.ConformerOracle(hp, t).stream(right, g["left"], g["drop"])
    n = 0
    for j, (ch, length, first) in enumerate(mel_chunks(mel, g)):
        print(f"stream right {right} chunk {j} frames {ch.shape[1]}{f16_note}", flush=True)
        got = s.step(ch, length)[0]
        want = o.step(ch, length)
        _same(got, want, (right, j))
        n += len(want)
    s.close()
    enc.close()
    return n


@pytest.mark.parametrize("right", [13, 6, 1, 0])
def test_stream_chunks_bit_exact(kern, orc, right):
    """Left context 28: 5 s are 63 rows, so the key ring (left + chunk rows)
    and the convolution ring wrap many times."""
    t = conformer_model(STREAM_TINY28, seed=33, pointwise_f16=True)
    n = _stream_case(kern, orc, STREAM_TINY28, t, right, 5.0, 61)
    assert n >= 60


@pytest.mark.parametrize("right,fuse,dw,gk", [(13, 0, -1, -1), (0, 0, -1, -1), (13, 3, -1, -1), (6, 3, -1, -1),
                                              (13, -1, 0, -1), (0, -1, 0, -1), (13, -1, -1, 3), (0, -1, -1, 3)])
def test_stream_chunks_fusions(kern, orc, right, fuse, dw, gk):
    """The chunk steps with every LayerNorm, GLU and cache copy in a launch
    of its own (CONF_FUSE=0), with the LayerNorms in the prologues of the
    K-split products too (CONF_FUSE=3), with the depthwise convolution's
    LayerNorm by a whole workgroup (CONF_DW=0) instead of one wave, and with
    every product on the LDS tiles (GEMM_KERNEL=3: their GLU and ring
    copies): the oracle's bits every way."""
    t = conformer_model(STREAM_TINY28, seed=33, pointwise_f16=True)
    with kern.tuned(CONF_FUSE=fuse, CONF_DW=dw, GEMM_KERNEL=gk):
        assert _stream_case(kern, orc, STREAM_TINY28, t, right, 3.0, 64, f" fuse {fuse} dw {dw} gk {gk}") >= 35


@pytest.mark.parametrize("right", [13, 0])
def test_stream_long_left_context(kern, orc, right):
    t = conformer_model(STREAM_TINY, seed=34, pointwise_f16=False)
    assert _stream_case(kern, orc, STREAM_TINY, t, right, 8.0, 62) >= 99


@pytest.mark.parametrize("rq,g8,right,thr", [(0, -1, 6, -1), (1, -1, 6, -1), (4, -1, 6, -1), (8, -1, 6, -1),
                                             (16, -1, 6, -1), (4, 0, 1, -1), (4, -1, 1, -1), (4, -1, 0, -1),
                                             (1, -1, 13, -1), (1, -1, 13, 256), (1, -1, 0, 512)])
def test_stream_attention_kernels(kern, orc, rq, g8, right, thr):
    """Each attention kernel form on the chunk steps: unstaged, and staged
    with 1, 4, 8 or 16 query rows per workgroup; at right contexts 1 and 0
    with each output of a few-row block by 8 lanes or by one thread
    (CONF_ATTN_G8=0); a row a workgroup on 256 or 512 threads
    (CONF_ATTN_THREADS) as well as 1024."""
    t = conformer_model(STREAM_TINY28, seed=39, pointwise_f16=True)
    with kern.tuned(CONF_ATTN_RQ=rq, CONF_ATTN_G8=g8, CONF_ATTN_THREADS=thr):
        assert _stream_case(kern, orc, STREAM_TINY28, t, right, 3.0, 63, f" rq {rq} g8 {g8} thr {thr}") >= 35


def test_stream_attention_staging_overflow(kern, orc):
    """A row a workgroup on 256 threads whose staged rows (up to 84 keys of
    a 64-wide head, 1344 float4s) outnumber the 1024 its registers hold:
    the rest is staged straight from memory, the same bits."""
    hp = dict(STREAM_TINY, heads=1)
    t = conformer_model(hp, seed=40, pointwise_f16=True)
    with kern.tuned(CONF_ATTN_RQ=1, CONF_ATTN_THREADS=256):
        assert _stream_case(kern, orc, hp, t, 13, 8.0, 66, " staging overflow") >= 99


def test_streams_together_equal_alone(kern, orc):
    """Three streams stepped together: each one's rows are those it gets
    alone (and the oracle's); the last chunks have different real frames."""
    hp = STREAM_TINY28
    t = conformer_model(hp, seed=35, pointwise_f16=True)
    right = 6
    g = stream_geom(hp, right)
    mels = [noise_mel(hp["n_mels"], seconds=3.0, seed=70 + i)[0] for i in range(3)]
    chunks = [mel_chunks(m, g) for m in mels]
    enc = ConformerEncoder(hp, t)
    together = ConformerStream(enc, right, batch=3)
    alone = [ConformerStream(enc, right) for _ in range(3)]
    orcs = [orc.ConformerOracle(hp, t).stream(right, g["left"], g["drop"]) for _ in range(3)]
    for j in range(len(chunks[0])):
        nf = chunks[0][j][0].shape[1]
        # the last chunk: every stream's frames, fewer of them real in two
        lengths = [nf, max(1, nf - 3), max(1, nf - 11)] if j == len(chunks[0]) - 1 else [nf] * 3
        print(f"streams chunk {j} frames {nf} lengths {lengths}", flush=True)
        batch = np.stack([c[j][0] for c in chunks])
        rows = together.step(batch, lengths)
        for b in range(3):
            one = alone[b].step(batch[b], lengths[b])[0]
            want = orcs[b].step(batch[b], lengths[b])
            _same(rows[b], one, (j, b, "alone"))
            _same(rows[b], want, (j, b, "oracle"))
    together.close()
    for a in alone:
        a.close()
    enc.close()


def test_stream_step_dev_matches_host(kern, orc):
    from gorelaxor_amd import hiprt
    hp = STREAM_TINY28
    t = conformer_model(hp, seed=36, pointwise_f16=True)
    g = stream_geom(hp, 13)
    mel, _, _ = noise_mel(hp["n_mels"], seconds=2.0, seed=80)
    enc = ConformerEncoder(hp, t)
    a, b = ConformerStream(enc, 13), ConformerStream(enc, 13)
    dout = hiprt.DeviceBuffer(g["chunk"] * hp["d"] * 4)
    for j, (ch, n, _) in enumerate(mel_chunks(mel, g)):
        print(f"step_dev chunk {j}", flush=True)
        dm = hiprt.DeviceBuffer.from_array(np.ascontiguousarray(ch, np.float32))
        lens = b.step_dev(dm.ptr, ch.shape[1], n, dout.ptr)
        got = dout.download(np.float32, (g["chunk"], hp["d"]))[:lens[0]]
        _same(got, a.step(ch, n)[0], j)
    a.close()
    b.close()
    enc.close()


def test_stream_errors(kern):
    t = conformer_model(STREAM_TINY28, seed=37)
    enc = ConformerEncoder(STREAM_TINY28, t)
    with pytest.raises(GrxError, match="wasn't trained for a right context of 5"):
        ConformerStream(enc, 5)
    s = ConformerStream(enc, 1)
    g = s.geom
    mel = np.zeros((STREAM_TINY28["n_mels"], g["mel_first"] + 64), np.float32)
    with pytest.raises(GrxError, match="more than the stream's"):
        s.step(mel, mel.shape[1])
    # a first chunk of one frame still gives one row
    assert len(s.step(mel[:, :1], 1)[0]) == 1
    with pytest.raises(GrxError, match="outside"):
        s.step(mel[:, :17], 18)
    s.close()
    enc.close()
    reg = ConformerEncoder(CONFORMER_TINY, conformer_model(CONFORMER_TINY, seed=38))
    with pytest.raises(GrxError, match="can't stream"):
        ConformerStream(reg, 13)
    reg.close()


@pytest.fixture(scope="module")
def nemotron():
    return conformer_model(NEMOTRON_STREAMING, seed=3, pointwise_f16=True)


@pytest.mark.parametrize("right,seconds,most", [(13, 8.0, 9), (0, 1.0, 14)])
def test_nemotron_shape_chunks_bit_exact(kern, orc, nemotron, right, seconds, most):
    """The M=14 and M=1 chunk steps at the full width and depth: at right
    context 13 the key ring (84 rows) wraps within the 8 s."""
    hp = NEMOTRON_STREAMING
    mel, _, _ = noise_mel(hp["n_mels"], seconds=seconds, seed=90)
    g = stream_geom(hp, right)
    enc = ConformerEncoder(hp, nemotron)
    s = ConformerStream(enc, right)
    o = orc.ConformerOracle(hp, nemotron).stream(right, g["left"], g["drop"])
    for j, (ch, n, _) in enumerate(mel_chunks(mel, g)[:most]):
        print(f"nemotron right {right} chunk {j}", flush=True)
        _same(s.step(ch, n)[0], o.step(ch, n), (right, j))
    s.close()
    enc.close()
