"""QSF loader (qstream_amd/host/qsf_loader.c) on the CPU: the CRC-32 of
src/format.c:11-34 against zlib (a library CRC-32 of the same polynomial)
and the reference's known answers (tests/test_core.c:57-71), and every
malformed-file rejection, which happens before the loader touches a GPU
(src/format.c:37-99, 146-180; layer records of src/engine.c:183-202)."""
from __future__ import annotations

import struct
import zlib

import numpy as np
import pytest

from qstream_amd import qsf_format as F


@pytest.fixture(scope="module")
def hip():
    from qstream_amd import qsf_hip
    qsf_hip.load()
    return qsf_hip


def test_crc32_known_answers(hip):
    assert hip.crc32(b"") == 0x00000000
    assert hip.crc32(b"123456789") == 0xCBF43926
    rng = np.random.default_rng(1)
    for n in (1, 7, 168, 4096, 100003):
        b = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert hip.crc32(b) == zlib.crc32(b) & 0xFFFFFFFF


def small_model(rng, hidden=256, vocab=300, bs=64):
    q4 = lambda r, c: F.quantize_matrix(F.gaussian(rng, (r, c), 0.02), F.Q4, bs)  # noqa: E731
    layers = []
    for _ in range(2):
        norm = F.gaussian(rng, hidden, 1.0).astype(np.float16).tobytes()
        layers.append([(F.T_ATTN_NORM_W, F.FP16, 1, hidden, norm),
                       (F.T_ATTN_Q, 0xFF, hidden, hidden, q4(hidden, hidden)),
                       (F.T_FFN_DOWN, F.Q3, hidden, 512,
                        F.quantize_matrix(F.gaussian(rng, (hidden, 512), 0.02), F.Q3, bs))])
    emb = (F.Q4, q4(vocab, hidden))
    return dict(hidden=hidden, heads=4, vocab=vocab, inter=512, layers=layers, quant_type=F.Q4,
                block_size=bs, embedding=emb, final_norm=np.ones(hidden, np.float16),
                output_head=q4(vocab, hidden))


def patch(path, off, fmt, *vals):
    b = bytearray(open(path, "rb").read())
    struct.pack_into(fmt, b, off, *vals)
    open(path, "wb").write(bytes(b))


def expect(hip, path, code, words):
    with pytest.raises(hip.QsfHipError) as e:
        hip.Model(str(path))
    msg = str(e.value)
    assert f"({code})" in msg, msg
    for w in words:
        assert w in msg, msg


def test_rejects_malformed_files(hip, tmp_path):
    rng = np.random.default_rng(2)
    kw = small_model(rng)
    base = tmp_path / "base.qsf"
    offs = F.write_qsf(str(base), **kw)
    raw = open(base, "rb").read()
    cases = [
        ("magic", lambda p: patch(p, 0, "<I", 0x12345678), 2, ["magic"]),
        ("version", lambda p: patch(p, 4, "<I", 2), 3, ["version"]),
        ("layers", lambda p: patch(p, 16, "<I", 0), 6, ["num_layers"]),
        ("vocab", lambda p: patch(p, 32, "<I", 50), 6, ["vocab"]),
        ("block", lambda p: patch(p, 60, "<I", 96), 6, ["block_size"]),
        ("heads", lambda p: patch(p, 24, "<I", 3), 6, ["num_heads"]),
        ("index", lambda p: patch(p, 64, "<Q", offs["size"] - 10), 2, ["layer index"]),
        ("lz4", lambda p: patch(p, offs["layer_index"] + 48 + 17, "<B", 1), 15, ["LZ4"]),
        ("past_layer", lambda p: patch(p, offs["layer_offsets"][0] + 24 + 512 + 12, "<I", 10 ** 6), 2,
         ["past the layer end"]),
        ("short_matrix", lambda p: patch(p, offs["layer_offsets"][1] + 24 + 512 + 8, "<I", 4096), 6,
         ["its matvec reads"]),
        ("truncated", lambda p: open(p, "wb").write(raw[:200]), 2, ["too small"]),
    ]
    for name, mutate, code, words in cases:
        p = tmp_path / f"{name}.qsf"
        p.write_bytes(raw)
        mutate(str(p))
        expect(hip, p, code, words)
    expect(hip, tmp_path / "missing.qsf", 1, ["cannot open"])


def test_embedding_span_is_what_the_upload_reads(hip, tmp_path):
    """The embedding is sized as its upload reads it, before any device
    work: the outlier table of a type-9 table (its count from the file),
    17-byte MXFP4 records at any block size, FP16 rows at the engine's
    stride of whole blocks (src/engine.c:718-721, src/quant.c:68-85).  A
    file shorter than that span is rejected, never read past its end."""
    rng = np.random.default_rng(3)
    hidden, vocab = 256, 300
    # type 9, the embedding last in the file, its outlier count past the end
    kw = small_model(rng, hidden=hidden, vocab=vocab)
    kw.update(final_norm=None, output_head=None,
              embedding=(F.Q2_OUTLIER, F.quantize_matrix(F.heavy_tail_weights(rng, vocab, hidden), F.Q2_OUTLIER, 64)))
    p = tmp_path / "emb9.qsf"
    offs = F.write_qsf(str(p), **kw)
    n_out = struct.unpack_from("<I", p.read_bytes(), offs["embedding"] + 32)[0]
    assert n_out > 0
    patch(str(p), offs["embedding"] + 32, "<I", 0xFFFFFFFF)
    expect(hip, p, 2, ["embedding data past the end"])
    # one outlier more than the file holds
    patch(str(p), offs["embedding"] + 32, "<I", n_out + 1)
    expect(hip, p, 2, ["embedding data past the end"])
    # type 11 at block 256: 132-byte blocks written where 17-byte records of 32 are read
    kw = small_model(rng, hidden=hidden, vocab=vocab, bs=256)
    kw.update(final_norm=None, output_head=None,
              embedding=(F.MXFP4, rng.integers(0, 256, vocab * 132, dtype=np.uint8).tobytes()))
    p = tmp_path / "emb11.qsf"
    F.write_qsf(str(p), **kw)
    expect(hip, p, 2, ["embedding data past the end"])
    # FP16 rows of 96 values with block 64: the engine reads rows of 128
    kw = small_model(rng, hidden=96, vocab=vocab)
    kw.update(final_norm=None, output_head=None,
              embedding=(F.FP16, F.gaussian(rng, (vocab, 96)).astype(np.float16).tobytes()))
    p = tmp_path / "emb7.qsf"
    F.write_qsf(str(p), **kw)
    expect(hip, p, 2, ["embedding data past the end"])
