"""A writer of whisper.cpp (ggml) model files for tests, in the layout
whisper/model.go:117-219 reads: magic, 11 int32 hyper-parameters, the mel
filter bank, the vocabulary, then tensors (n_dims, name length, type, dims
with ne[0] the row length, name, data) until the end of the file.  Also
numpy encoders and decoders of the block formats used in the tests
(dequantBlock, model.go:449-492)."""
from __future__ import annotations

import struct

import numpy as np

MAGIC = 0x67676D6C
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0 = 0, 1, 2, 3, 6, 7, 8


def whisper_file_hparams(dec_hp: dict, n_mels: int = 80, n_audio_layer: int = 1, ftype: int = 7) -> list:
    """The 11 header ints of a file whose decoder is `dec_hp` (its n_audio_ctx
    must be 1500 and n_vocab 51864..60000, as the loader requires)."""
    st = dec_hp["n_state"]
    return [dec_hp["n_vocab"], dec_hp["n_audio_ctx"], st, dec_hp["n_head"], n_audio_layer, dec_hp["n_text_ctx"], st,
            dec_hp["n_head"], dec_hp["n_layer"], n_mels, ftype]


def q4_0_blocks(rng: np.random.Generator, n: int) -> tuple[np.ndarray, np.ndarray]:
    """Random Q4_0 data for n values: (bytes, float32 values d*(q-8))."""
    nb = n // 32
    d = (np.abs(rng.standard_normal(nb)) * 0.01).astype(np.float16)
    q = rng.integers(0, 16, size=(nb, 32), dtype=np.int64)
    blk = np.zeros((nb, 18), np.uint8)
    blk[:, :2] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 2:] = (q[:, :16] | q[:, 16:] << 4).astype(np.uint8)
    vals = ((q - 8).astype(np.float32) * d.astype(np.float32)[:, None]).reshape(-1)
    return blk.reshape(-1), vals


def q5_1_blocks(rng: np.random.Generator, n: int) -> tuple[np.ndarray, np.ndarray]:
    """Random Q5_1 data for n values: (bytes, float32 values d*q + m with q
    the 5-bit value whose fifth bit is bit j of qh)."""
    nb = n // 32
    d = (np.abs(rng.standard_normal(nb)) * 0.01).astype(np.float16)
    m = (rng.standard_normal(nb) * 0.05).astype(np.float16)
    q = rng.integers(0, 32, size=(nb, 32), dtype=np.int64)
    qh = np.zeros(nb, np.uint32)
    for j in range(32):
        qh |= ((q[:, j] >> 4) & 1).astype(np.uint32) << np.uint32(j)
    blk = np.zeros((nb, 24), np.uint8)
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 2:4] = m.view(np.uint8).reshape(nb, 2)
    blk[:, 4:8] = qh.view(np.uint8).reshape(nb, 4)
    blk[:, 8:] = ((q[:, :16] & 15) | (q[:, 16:] & 15) << 4).astype(np.uint8)
    vals = (q.astype(np.float32) * d.astype(np.float32)[:, None] + m.astype(np.float32)[:, None]).reshape(-1)
    return blk.reshape(-1), vals


def tensor_record(name: str, typ: int, ne: list, data: np.ndarray) -> bytes:
    nb = name.encode()
    return (struct.pack("<iii", len(ne), len(nb), typ) + struct.pack(f"<{len(ne)}i", *ne) + nb +
            np.ascontiguousarray(data).tobytes())


def write(path, hparams: list, tensors: list, n_mels: int | None = None, n_words: int = 3, magic: int = MAGIC,
          truncate: int = 0) -> None:
    """tensors: (name, type, ne, data) in file order; `truncate` drops that
    many bytes from the end."""
    n_mels = hparams[9] if n_mels is None else n_mels
    out = [struct.pack("<I", magic), struct.pack("<11i", *hparams), struct.pack("<ii", n_mels, 201),
           np.zeros(n_mels * 201, np.float32).tobytes(), struct.pack("<i", n_words)]
    for i in range(n_words):
        w = f"w{i}".encode()
        out.append(struct.pack("<i", len(w)) + w)
    out += [tensor_record(*t) for t in tensors]
    blob = b"".join(out)
    if truncate:
        blob = blob[:-truncate]
    with open(path, "wb") as f:
        f.write(blob)
