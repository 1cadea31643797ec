"""The benchmark's CPU baseline - the reference's int8 product with the
VNNI tile kernel and its task split (oracle/grx_vnni.cc, restating
internal/kern/q8int.go:35-223 and vnni_amd64.s) - gives the oracle's bits:
odd sizes (partial row tiles and panels, q8int_test.go / odd_test.go
shapes), the task split at several thread counts, a zero block, and the
ring loop the bench times."""
import numpy as np
import pytest

from gorelaxor_amd.synth import q8_weight


@pytest.fixture(scope="module")
def vnni(orc):
    if orc.vnni_kind() == 0:
        pytest.skip("this CPU has neither AVX512-VNNI nor AVX-VNNI")
    return orc


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("m", [1, 2, 5, 6, 7, 16, 17, 23, 49])
@pytest.mark.parametrize("n", [1, 3, 16, 17, 33])
def test_odd_sizes_equal_the_oracle(vnni, m, n):
    rng = np.random.default_rng(m * 100 + n)
    for k in (32, 96):
        w8 = q8_weight(rng, n, k)
        x = rng.standard_normal((m, k)).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32) if n % 2 else None
        want = vnni.matmul_q8_int(x, w8, n, k, b)
        vw = vnni.VnniWeight(w8, n, k)
        for threads in (1, 3, 8):
            assert np.array_equal(_bits(vnni.vnni_matmul(x, vw, b, threads=threads)), _bits(want)), (m, n, k, threads)


def test_large_and_zero_blocks(vnni):
    rng = np.random.default_rng(7)
    m, n, k = 300, 1024, 1024  # the reference benchmark's 300 x 1024 x 1024
    w8 = q8_weight(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[3, 64:96] = 0.0  # a block of zeros: scale 0, bytes 128
    want = vnni.matmul_q8_int(x, w8, n, k)
    got = vnni.vnni_matmul(x, vnni.VnniWeight(w8, n, k), threads=8)
    assert np.array_equal(_bits(got), _bits(want))


def test_ring_loop(vnni):
    rng = np.random.default_rng(9)
    n, k, count = 64, 256, 5
    w8 = q8_weight(rng, n * count, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    panels, per = vnni.vnni_pack_many(w8, count, n, k)
    y = np.zeros(count * n, np.float32)
    vnni.vnni_ring(y, x, panels, per, count, n, k, 2, 2)
    src = n * (k // 32) * 34
    for i in range(count):
        want = vnni.matmul_q8_int(x, w8[i * src:(i + 1) * src], n, k)[0]
        assert np.array_equal(_bits(y[i * n:(i + 1) * n]), _bits(want)), i


def test_graphs_on_vnni_products_give_the_same_bits(orc):
    """The CPU baselines run the oracle's graphs with every int8 product on
    the VNNI restatement (oracle.vnni_products, 1 and 4 threads): the
    outputs are the scalar oracle's bit for bit (whisper steps, the pocket
    prefix and frames, a conformer encode)."""
    import pytest

    if orc.vnni_kind() == 0:
        pytest.skip("no VNNI on this processor")
    from gorelaxor_amd.synth import (CONFORMER_TINY, POCKET_TTS_TINY, WHISPER_TINY_TEST, conformer_model,
                                     encoder_output, pocket_inputs, pocket_model, whisper_model)

    def same(a, b):
        return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))

    hp = dict(WHISPER_TINY_TEST)
    t = whisper_model(hp, seed=4)
    enc = encoder_output(hp, seed=5)

    def whisper_run():
        ref = orc.WhisperOracle(hp, t)
        ref.set_encoder_output(enc)
        return [ref.decode([1, 2, 3])] + [ref.decode([k]) for k in (7, 8, 9)]

    php = dict(POCKET_TTS_TINY)
    pt = pocket_model(php, seed=6)
    x, lat = pocket_inputs(php, 3, prefix=9, seed=7)

    def pocket_run():
        ref = orc.PocketOracle(php, pt)
        return [ref.run(x)] + [ref.step(lat[k])[0] for k in range(3)]

    chp = dict(CONFORMER_TINY)
    ct = conformer_model(chp, seed=8)
    mel = np.random.default_rng(9).standard_normal((1, 48, chp["n_mels"])).astype(np.float32)

    def conformer_run():
        return [orc.ConformerOracle(chp, ct).encode(mel, 48)[0]]

    for run in (whisper_run, pocket_run, conformer_run):
        want = run()
        for threads in (1, 4):
            with orc.vnni_products(threads):
                got = run()
            assert all(same(g, w) for g, w in zip(got, want)), (run.__name__, threads)
