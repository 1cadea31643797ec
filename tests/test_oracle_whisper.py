"""Pins the oracle's whisper-shaped Q8_0 decoder (whisper/decoder.go:33-140
with int8-route products) without a GPU: an independent float64 restatement
of the graph bounds it, and incremental decoding equals decoding the prompt
at once, bit for bit (the reference decodes the prompt in one call,
whisper/transcribe.go:190, then one token per call, :245)."""
import numpy as np
import pytest

from gorelaxor_amd.synth import WHISPER_TINY_TEST, encoder_output, q8_dequant, whisper_model


def _ref_decode(hp, t, enc, tokens):
    """float64 decoder with the exact Q8_0 weights and unrounded activations:
    the textbook graph (pre-LN blocks, causal self-attention, cross-attention,
    tanh-GELU MLP, tied logits)."""
    st, nh = hp["n_state"], hp["n_head"]
    hd = st // nh
    W = lambda n, r, c: q8_dequant(t[n], r, c).astype(np.float64)  # noqa: E731
    V = lambda n: t[n].astype(np.float64)  # noqa: E731

    def ln(x, w, b):
        mu = x.mean(-1, keepdims=True)
        return (x - mu) / np.sqrt(x.var(-1, keepdims=True) + 1e-5) * w + b

    def attn(q, k, v):
        s = (q.reshape(-1, nh, hd).transpose(1, 0, 2) @ k.reshape(-1, nh, hd).transpose(1, 2, 0)) / np.sqrt(hd)
        return s, v.reshape(-1, nh, hd).transpose(1, 0, 2)

    emb = W("decoder.token_embedding.weight", hp["n_vocab"], st)
    pos = V("decoder.positional_embedding").reshape(hp["n_text_ctx"], st)
    n = len(tokens)
    x = emb[tokens] + pos[:n]
    e = enc.reshape(hp["n_audio_ctx"], st).astype(np.float64)
    for i in range(hp["n_layer"]):
        p = f"decoder.blocks.{i}."
        h = ln(x, V(p + "attn_ln.weight"), V(p + "attn_ln.bias"))
        q = h @ W(p + "attn.query.weight", st, st).T + V(p + "attn.query.bias")
        k = h @ W(p + "attn.key.weight", st, st).T
        v = h @ W(p + "attn.value.weight", st, st).T + V(p + "attn.value.bias")
        s, vh = attn(q, k, v)
        s = s + np.triu(np.full((n, n), -np.inf), 1)
        a = np.exp(s - s.max(-1, keepdims=True))
        a /= a.sum(-1, keepdims=True)
        o = (a @ vh).transpose(1, 0, 2).reshape(n, st)
        x = x + o @ W(p + "attn.out.weight", st, st).T + V(p + "attn.out.bias")
        h = ln(x, V(p + "cross_attn_ln.weight"), V(p + "cross_attn_ln.bias"))
        q = h @ W(p + "cross_attn.query.weight", st, st).T + V(p + "cross_attn.query.bias")
        k = e @ W(p + "cross_attn.key.weight", st, st).T
        v = e @ W(p + "cross_attn.value.weight", st, st).T + V(p + "cross_attn.value.bias")
        s, vh = attn(q, k, v)
        a = np.exp(s - s.max(-1, keepdims=True))
        a /= a.sum(-1, keepdims=True)
        o = (a @ vh).transpose(1, 0, 2).reshape(n, st)
        x = x + o @ W(p + "cross_attn.out.weight", st, st).T + V(p + "cross_attn.out.bias")
        h = ln(x, V(p + "mlp_ln.weight"), V(p + "mlp_ln.bias"))
        f = h @ W(p + "mlp.0.weight", 4 * st, st).T + V(p + "mlp.0.bias")
        f = 0.5 * f * (1 + np.tanh(np.sqrt(2 / np.pi) * f * (1 + 0.044715 * f * f)))
        x = x + f @ W(p + "mlp.2.weight", st, 4 * st).T + V(p + "mlp.2.bias")
    h = ln(x[-1], V("decoder.ln.weight"), V("decoder.ln.bias"))
    return h @ emb.T


@pytest.fixture(scope="module")
def tiny(orc):
    hp = dict(WHISPER_TINY_TEST)
    t = whisper_model(hp, seed=3)
    enc = encoder_output(hp, seed=4)
    return hp, t, enc


def test_oracle_decoder_vs_float64(orc, tiny):
    """The oracle's logits stay within the error Q8_0 activation rounding
    allows of the float64 graph (relative RMS), at every position."""
    hp, t, enc = tiny
    m = orc.WhisperOracle(hp, t)
    m.set_encoder_output(enc)
    toks = [5, 17, 3, 999, 42, 0, 7]
    for n in range(1, len(toks) + 1):
        m.reset()
        got = m.decode(toks[:n])
        want = _ref_decode(hp, t, enc, np.array(toks[:n]))
        rel = np.sqrt(((got - want) ** 2).mean() / (want ** 2).mean())
        assert rel < 0.03, (n, rel)


def test_oracle_incremental_equals_prompt(orc, tiny):
    """Decoding tokens one call at a time gives the logits of decoding them in
    one call, bit for bit, and the cache holds the same keys and values."""
    hp, t, enc = tiny
    a = orc.WhisperOracle(hp, t)
    a.set_encoder_output(enc)
    b = orc.WhisperOracle(hp, t)
    b.set_encoder_output(enc)
    toks = [1, 2, 3, 4, 5]
    la = a.decode(toks)
    for tk in toks:
        lb = b.decode([tk])
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    assert a.n == b.n == 5
    for i in range(hp["n_layer"]):
        assert np.array_equal(a.self_k[i], b.self_k[i]) and np.array_equal(a.self_v[i], b.self_v[i])


def test_oracle_greedy_and_context_limit(orc, tiny):
    hp, t, enc = tiny
    m = orc.WhisperOracle(hp, t)
    m.set_encoder_output(enc)
    toks = m.greedy([1, 2, 3, 4], 10)
    assert toks.shape == (11,) and m.n == 14
    # the greedy loop is decode + argmax fed back
    m.reset()
    lg = m.decode([1, 2, 3, 4])
    seq = [int(np.argmax(lg))]
    for _ in range(10):
        lg = m.decode([seq[-1]])
        seq.append(orc.argmax(lg))
    assert list(toks) == seq
    m.reset()
    with pytest.raises(ValueError):
        m.decode(list(range(hp["n_text_ctx"] + 1)))
