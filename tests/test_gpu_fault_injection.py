"""The library's error paths under injected out-of-memory failures
(grx_debug_fail_alloc_after): for each model, every device or pinned
allocation its set-up makes (create, tensors, the first use that moves
them to the device) is made to fail in turn.  Each failure must come back
as GRX_ENOMEM from the call that made the allocation; the same call made
again (after it) must succeed and the model then give exactly what a
clean build gives; destroying it must return all device memory.  The
reference reaches its own error paths through panics turned into errors
(conformer/robust_test.go:16-27, conformer/model.go:282-289)."""
import numpy as np
import pytest

from gorelaxor_amd import GrxError, _lib, hiprt

pytestmark = pytest.mark.gpu

ENOMEM = -4


def _arm(n):
    _lib.lib().grx_debug_fail_alloc_after(n)


def _left():
    return _lib.lib().grx_debug_alloc_countdown()


def _close(objs):
    for k in reversed(list(objs)):
        if hasattr(objs[k], "close"):
            objs[k].close()
    objs.clear()


def _sweep(steps, result, limit=600):
    """steps: callables building the model into a dict, in order; result:
    the finished model's output (an array).  Two rounds over every
    allocation: the first lets the HIP runtime's own pools reach their size,
    the second must end with the device memory it started with.  Returns
    the allocations the build makes."""
    objs = {}
    try:
        for st in steps:
            st(objs)
        want = np.ascontiguousarray(result(objs))
    finally:
        _close(objs)
    n1 = _round(steps, result, want, limit)
    hiprt.synchronize()
    base = hiprt.mem_free()
    n2 = _round(steps, result, want, limit)
    hiprt.synchronize()
    assert n1 == n2
    assert hiprt.mem_free() == base, f"device memory not returned: {base - hiprt.mem_free()} bytes"
    return n1


def _round(steps, result, want, limit):
    objs = {}
    n = 0
    free0 = hiprt.mem_free()
    while True:
        assert n < limit, "the build never finished"
        failed_at = None
        _arm(n)
        try:
            for k, st in enumerate(steps):
                try:
                    st(objs)
                except GrxError as e:
                    assert e.status == ENOMEM, (n, k, str(e))
                    assert _left() == -1, (n, k, "failed, but not by the injected allocation")
                    failed_at = k
                    break
            left = _left()
            _arm(-1)
            if failed_at is not None:
                for st in steps[failed_at:]:  # the failed call again, and the rest
                    try:
                        st(objs)
                    except GrxError as e:
                        # a tensor kept by the failed call; or the last tensor,
                        # kept before the set-up it started failed (the next
                        # use retries that set-up)
                        if "given twice" not in str(e) and "complete already" not in str(e):
                            raise
            got = np.ascontiguousarray(result(objs))
            assert got.shape == want.shape and np.array_equal(got.view(np.uint8), want.view(np.uint8)), n
        finally:
            _arm(-1)
            _close(objs)
        hiprt.synchronize()
        free = hiprt.mem_free()
        if free != free0:
            print(f"  allocation {n} (step {failed_at}): free device memory {free - free0:+d} bytes")
            free0 = free
        if failed_at is None:
            assert left >= 0
            break
        n += 1
    return n


def test_conformer_encode_and_stream():
    from gorelaxor_amd.conformer import ConformerEncoder, ConformerStream, mel_chunks, stream_geom
    from gorelaxor_amd.synth import CONFORMER_TINY, conformer_model, noise_mel

    hp = dict(CONFORMER_TINY, att_style="chunked_limited", att_left=28, att_right=6,
              context_choices=[(28, 6), (28, 1)], conv_left=8, conv_right=0, conv_norm="layer_norm")
    t = conformer_model(hp, seed=51)
    mel, frames, valid = noise_mel(hp["n_mels"], seconds=1.0, seed=52)
    chunks = mel_chunks(mel, stream_geom(hp, 6))

    def create(o):
        o["enc"] = ConformerEncoder(hp)

    def tensors(o):
        for k, v in t.items():
            o["enc"].set_tensor(k, v)

    def encode(o):
        o["out"] = o["enc"].encode(mel, valid)[0]

    def stream(o):
        o["s"] = ConformerStream(o["enc"], 6)

    def steps(o):
        o["rows"] = np.concatenate([o["s"].step(c, n)[0] for c, n, _ in chunks])

    n = _sweep([create, tensors, encode, stream, steps],
               lambda o: np.concatenate([o["out"].ravel(), o["rows"].ravel()]))
    print("conformer allocations", n)
    assert n > 40


def test_whisper_decode():
    from gorelaxor_amd.synth import WHISPER_TINY_TEST, encoder_output, whisper_model
    from gorelaxor_amd.whisper import WhisperDecoder

    hp = dict(WHISPER_TINY_TEST)
    t = whisper_model(hp, seed=53)
    enc = encoder_output(hp, seed=54)

    def create(o):
        o["dec"] = WhisperDecoder(hp)

    def tensors(o):
        for k, v in t.items():
            o["dec"].set_tensor(k, v)

    def cross(o):
        o["dec"].set_encoder_output(enc)

    def greedy(o):
        o["tok"] = o["dec"].greedy([1, 2, 3], 6)

    n = _sweep([create, tensors, cross, greedy], lambda o: o["tok"])
    print("whisper allocations", n)
    assert n > 20


def test_pocket_frames_and_speak():
    from gorelaxor_amd.pocket import PocketLM
    from gorelaxor_amd.synth import POCKET_FLOW_TINY, POCKET_TTS_TINY, pocket_flow_model, pocket_inputs, \
        pocket_model

    hp, fhp = dict(POCKET_TTS_TINY), dict(POCKET_FLOW_TINY)
    t = pocket_model(hp, seed=55)
    ft = pocket_flow_model(hp, fhp, seed=56)
    x, _ = pocket_inputs(hp, 1, prefix=5, seed=57)
    noise = np.random.default_rng(58).standard_normal((4, hp["ldim"])).astype(np.float32)

    def create(o):
        o["lm"] = PocketLM(hp)

    def tensors(o):
        for k, v in t.items():
            o["lm"].set_tensor(k, v)
        o["lm"].flow_init(fhp["dim"], fhp["depth"], fhp["steps"])
        for k, v in ft.items():
            o["lm"].set_tensor(k, v)

    def run(o):
        o["h"] = o["lm"].run(x)

    def speak(o):
        o["lat"], o["eos"] = o["lm"].speak(noise)

    n = _sweep([create, tensors, run, speak],
               lambda o: np.concatenate([o["h"].ravel(), o["lat"].ravel(), o["eos"].ravel()]))
    print("pocket allocations", n)
    assert n > 30


def test_rnnt_decode():
    from gorelaxor_amd.rnnt import TransducerDecoder
    from gorelaxor_amd.synth import RNNT_TINY, rnnt_encoder_output, rnnt_model

    hp = dict(RNNT_TINY)
    t = rnnt_model(hp, seed=59)
    enc = rnnt_encoder_output(hp, 20, seed=60)

    def create(o):
        o["dec"] = TransducerDecoder(hp)

    def tensor(name):
        def f(o):
            o["dec"].set_tensor(name, t[name])
        return f

    def state(o):
        o["st"] = o["dec"].new_state()

    def decode(o):
        toks = o["dec"].decode(enc, o["st"])
        o["toks"] = np.array([(k.ID, k.Frame, k.Duration) for k in toks], np.int64).ravel()

    n = _sweep([create] + [tensor(k) for k in t] + [state, decode], lambda o: o["toks"])
    print("rnnt allocations", n)
    assert n > 10


def test_mimi_decode():
    from gorelaxor_amd.mimi import MimiDecoder
    from gorelaxor_amd.synth import MIMI_TINY, mimi_latents, mimi_model

    hp = dict(MIMI_TINY)
    t = mimi_model(hp, seed=61, q8=True)
    lat = mimi_latents(hp, 6, seed=62)

    def create(o):
        o["dec"] = MimiDecoder(hp, max_latents=2)

    def tensor(name):  # each tensor goes to the device as it is set
        def f(o):
            o["dec"].set_tensor(name, t[name])
        return f

    def decode(o):
        o["pcm"] = np.concatenate([o["dec"].decode(lat[i:i + 2]) for i in range(0, 6, 2)])

    n = _sweep([create] + [tensor(k) for k in t] + [decode], lambda o: o["pcm"])
    print("mimi allocations", n)
    assert n > 10


def test_mimi_from_gguf(tmp_path):
    """grx_mimi_load_gguf's done() path: each allocation of the load (and of
    the first decode) fails in turn."""
    from gorelaxor_amd.mimi import MimiDecoder
    from gorelaxor_amd.synth import MIMI_TINY, mimi_latents, mimi_model
    from tests.test_gpu_mimi_load import _write

    hp = dict(MIMI_TINY)
    t = mimi_model(hp, seed=63, q8=True)
    p = _write(tmp_path / "m.gguf", hp, t)
    lat = mimi_latents(hp, 2, seed=64)

    def load(o):
        o["dec"] = MimiDecoder.from_gguf(p, max_latents=2)

    def decode(o):
        o["pcm"] = o["dec"].decode(lat)

    n = _sweep([load, decode], lambda o: o["pcm"])
    print("mimi gguf allocations", n)
    assert n > 10


def test_pocket_from_gguf(tmp_path):
    """grx_pocket_load_gguf: each allocation of the load and the first run
    fails in turn; then a voice state (grx_pocket_state_create and
    grx_pocket_set_state)."""
    from gorelaxor_amd.pocket import PocketLM
    from gorelaxor_amd.synth import POCKET_TTS_TINY, pocket_inputs, pocket_model
    from tests.test_gpu_pocket_load import _write

    hp = dict(POCKET_TTS_TINY)
    t = pocket_model(hp, seed=65)
    p = _write(tmp_path / "p.gguf", hp, t)
    x, _ = pocket_inputs(hp, 1, prefix=4, seed=66)
    rng = np.random.default_rng(67)
    kv = rng.standard_normal((2, hp["n_layer"], 7, hp["d"])).astype(np.float32)

    def load(o):
        o["lm"] = PocketLM.from_gguf(p, max_pos=hp["max_pos"])

    def voice(o):
        o["v"] = o["lm"].make_state(kv[0], kv[1])

    def run(o):
        o["lm"].set_state(o["v"])
        o["h"] = o["lm"].run(x)

    n = _sweep([load, voice, run], lambda o: o["h"])
    print("pocket gguf allocations", n)
    assert n > 10


def test_whisper_streams():
    """grx_whisper_create_streams (two streams sharing one window) and the
    device loop's buffers."""
    from gorelaxor_amd.synth import WHISPER_TINY_TEST, encoder_output, whisper_model
    from gorelaxor_amd.whisper import WhisperDecoder

    hp = dict(WHISPER_TINY_TEST)
    t = whisper_model(hp, seed=68)
    enc = encoder_output(hp, seed=69)

    def create(o):
        o["dec"] = WhisperDecoder(hp, streams=2)

    def tensors(o):
        for k, v in t.items():
            o["dec"].set_tensor(k, v)

    def cross(o):
        o["dec"].set_encoder_output_stream(0, enc)
        o["dec"].share_encoder_output(1, 0)

    def greedy(o):
        o["tok"] = o["dec"].greedy_streams([[1, 2, 3], [4, 5, 6]], 5)

    n = _sweep([create, tensors, cross, greedy], lambda o: o["tok"])
    print("whisper streams allocations", n)
    assert n > 20
