"""The QSF container this build writes (qsf_format.write_qsf) against
QStream's own reader: src/format.c, src/file_access.c and src/error.c
compiled from the reference tree into oracle/_ref (oracle/Makefile), with
the on-disk structs laid out by the reference's headers
(include/qsf/types.h:185-312) as its compiler lays them out.

For files of several shapes (per-tensor overrides, outlier types, FP16
vectors, separate and tied heads, an MoE layer of MXFP4 experts) the
reference's qsf_model_load returns QSF_OK with no warning, every header
field it holds is the value written, every layer-index entry points at the
layer's records, qsf_decompress_layer returns that span with its CRC
verified, and the tensor records, embedding and final section are found
where the engine looks for them (src/engine.c:183-202, 709-737, 664-679,
1200-1226).  tests/test_gpu_loader.py holds this build's loader to the
same reference parse on the GPU."""
from __future__ import annotations

import struct
import zlib

import numpy as np
import pytest

from qstream_amd import qsf_format as F
from tests import container_models as CM


@pytest.fixture(scope="module")
def rc():
    from oracle.oracle import ref_container
    r = ref_container()
    if r is None:
        pytest.skip("oracle/_ref not built (reference sources absent)")
    return r


# struct field -> struct format of its type (the sizes come from the reference)
_HEADER_FIELDS = {
    "magic": "I", "version": "I", "header_size": "I", "arch": "I", "num_layers": "I", "hidden_dim": "I",
    "num_heads": "I", "num_kv_heads": "I", "vocab_size": "I", "max_seq_len": "I", "intermediate_dim": "I",
    "head_dim": "I", "quant_type": "B", "activation": "B", "norm_type": "B", "pos_enc_type": "B",
    "rope_theta": "f", "norm_epsilon": "f", "block_size": "I", "layer_index_offset": "Q",
    "embedding_offset": "Q", "final_offset": "Q", "tokenizer_offset": "Q", "has_bias": "B", "ffn_type": "B",
    "attn_type": "B", "weight_tying": "B", "tie_word_embeddings": "I", "total_file_size": "Q",
    "header_crc32": "I", "endian_marker": "B", "num_experts": "B", "num_active_experts": "B",
    "moe_norm_topk": "B", "expert_intermediate_dim": "I"}


def _get(layout, struct_name, fields, buf, base=0):
    """Fields of a packed struct at buf[base:], at the reference's offsets."""
    return {f: struct.unpack_from("<" + t, buf, base + layout[f"{struct_name}.{f}"])[0]
            for f, t in fields.items()}


def _written(kw, offs, size):
    """Header values write_qsf was asked for (zero defaults as written)."""
    tied = kw.get("tied", False)
    return dict(magic=0x51534631, version=1, header_size=256, arch=1, num_layers=len(kw["layers"]),
                hidden_dim=kw["hidden"], num_heads=kw["heads"], num_kv_heads=kw.get("kv_heads", 0),
                vocab_size=kw["vocab"], max_seq_len=4096, intermediate_dim=kw["inter"],
                head_dim=kw.get("head_dim", 0), quant_type=kw["quant_type"], activation=kw.get("activation", 2),
                norm_type=kw.get("norm_type", 2), pos_enc_type=kw.get("pos_enc", 1),
                rope_theta=np.float32(kw.get("rope_theta", 10000.0)), norm_epsilon=np.float32(kw.get("eps", 1e-5)),
                block_size=kw.get("block_size", 64), layer_index_offset=offs["layer_index"],
                embedding_offset=offs["embedding"], final_offset=offs["final"], tokenizer_offset=0,
                has_bias=0, ffn_type=kw.get("ffn_type", 1), attn_type=0, weight_tying=int(tied),
                tie_word_embeddings=int(tied), total_file_size=size, endian_marker=1,
                num_experts=kw.get("num_experts", 0), num_active_experts=kw.get("num_active_experts", 0),
                moe_norm_topk=kw.get("moe_norm_topk", 0), expert_intermediate_dim=kw.get("expert_dim", 0))


def test_reference_struct_sizes(rc):
    """The packed sizes the on-disk format is defined by (types.h:185-312)."""
    L = rc.layout
    assert (L["QSFHeader"], L["QSFLayerIndex"], L["QSFTensorHeader"], L["QSFEmbeddingHeader"],
            L["QSFFinalHeader"], L["QSFOutlierEntry"]) == (256, 48, 24, 32, 16, 6)
    # the header CRC covers the bytes before its own field (src/format.c:129)
    assert L["QSFHeader.header_crc32"] == 168


def test_loader_rejection_offsets_are_the_reference_fields(rc):
    """The header offsets tests/test_loader.py patches to provoke each
    rejection are the reference's fields of those names."""
    L = rc.layout
    assert [L[f"QSFHeader.{f}"] for f in ("magic", "version", "num_layers", "vocab_size", "block_size",
                                          "num_heads", "layer_index_offset")] == [0, 4, 16, 32, 60, 24, 64]
    assert L["QSFLayerIndex.compression_type"] == 17 and L["QSFTensorHeader.data_size"] == 12


@pytest.mark.parametrize("name", ["dense", "dense_tied", "outlier_tied", "moe"])
def test_reference_reader_parses_written_file(rc, tmp_path, capfd, name):
    kw = CM.all_models()[name]
    path = tmp_path / f"{name}.qsf"
    offs = F.write_qsf(str(path), **kw)
    raw = path.read_bytes()
    capfd.readouterr()
    got = rc.load(str(path))
    err = capfd.readouterr().err
    assert got["rc"] == 0, got["error"]
    assert "[WARN]" not in err, err              # header CRC, file size, layer bounds, layer CRCs
    L = rc.layout

    # header, as the reference holds it
    h = _get(L, "QSFHeader", _HEADER_FIELDS, got["header"])
    assert h.pop("header_crc32") == zlib.crc32(raw[:168]) & 0xFFFFFFFF
    assert h == _written(kw, offs, len(raw))
    # derived values (src/format.c:145-162)
    assert got["head_dim"] == kw["hidden"] // kw["heads"]
    assert got["num_kv_heads"] == (kw.get("kv_heads") or kw["heads"])
    assert got["weight_tied"] == int(kw.get("tied", False))
    assert got["is_gated_ffn"] == int(kw.get("ffn_type", 1) == 1)
    assert got["uses_rope"] == int(kw.get("pos_enc", 1) == 1)
    assert got["file_size"] == len(raw)

    # layer index -> layer records, walked as src/engine.c:183-202 does
    li_fields = {"offset": "Q", "compressed_size": "I", "decompressed_size": "I", "quant_type": "B",
                 "compression_type": "B", "num_tensors": "H", "crc32_compressed": "I",
                 "crc32_decompressed": "I"}
    th_fields = {"tensor_type": "H", "quant_type": "B", "data_layout": "B", "rows": "I", "cols": "I",
                 "data_size": "I", "num_outliers": "I"}
    for i, recs in enumerate(kw["layers"]):
        e = _get(L, "QSFLayerIndex", li_fields, got["layer_index"], i * L["QSFLayerIndex"])
        assert e["offset"] == offs["layer_offsets"][i] == got["layer_data_off"][i]
        data = raw[e["offset"]:e["offset"] + e["compressed_size"]]
        assert e["compressed_size"] == e["decompressed_size"] == sum(L["QSFTensorHeader"] + len(r[4])
                                                                     for r in recs)
        assert (e["quant_type"], e["compression_type"], e["num_tensors"]) == (kw["quant_type"], 0, len(recs))
        assert e["crc32_compressed"] == e["crc32_decompressed"] == zlib.crc32(data) & 0xFFFFFFFF
        p = 0
        for ttype, qt, rows, cols, payload in recs:
            t = _get(L, "QSFTensorHeader", th_fields, data, p)
            assert t == dict(tensor_type=ttype, quant_type=qt, data_layout=0, rows=rows, cols=cols,
                             data_size=len(payload), num_outliers=0)
            p += L["QSFTensorHeader"]
            assert data[p:p + len(payload)] == bytes(payload)
            p += t["data_size"] + t["num_outliers"] * L["QSFOutlierEntry"]
        assert p == len(data)

    # embedding, where the engine's lookup reads it (src/engine.c:709-737)
    eqt, epay = kw["embedding"]
    eo = h["embedding_offset"]
    eh = _get(L, "QSFEmbeddingHeader", {"quant_type": "I", "compressed_size": "I", "num_vectors": "I",
                                        "embedding_dim": "I", "compression_type": "B", "crc32": "I",
                                        "num_chunks": "I", "chunk_size": "I"}, raw, eo)
    assert eh == dict(quant_type=eqt, compressed_size=0, num_vectors=kw["vocab"], embedding_dim=kw["hidden"],
                      compression_type=0, crc32=zlib.crc32(bytes(epay)) & 0xFFFFFFFF, num_chunks=1,
                      chunk_size=kw["vocab"])
    d0 = eo + L["QSFEmbeddingHeader"]
    assert raw[d0:d0 + len(epay)] == bytes(epay)

    # final section: norm weights, then the separate head (src/engine.c:403-420, 664-679)
    fo = h["final_offset"]
    fh = _get(L, "QSFFinalHeader", {"output_head_type": "I", "final_norm_size": "I", "output_head_size": "I",
                                    "crc32": "I"}, raw, fo)
    norm = np.asarray(kw["final_norm"], np.float16).tobytes()
    head = b"" if kw.get("tied") or kw.get("output_head") is None else bytes(kw["output_head"])
    assert fh == dict(output_head_type=int(kw.get("tied", False)), final_norm_size=len(norm),
                      output_head_size=len(head), crc32=zlib.crc32(norm + head) & 0xFFFFFFFF)
    f0 = fo + L["QSFFinalHeader"]
    assert raw[f0:f0 + len(norm)] == norm and raw[f0 + len(norm):f0 + len(norm) + len(head)] == head


def test_reference_reader_flags_what_ours_flags(rc, tmp_path, capfd):
    """A wrong layer CRC and a wrong total size are warnings in both readers
    (src/format.c:129-141, 226-233), not errors; a bad magic is an error."""
    kw = CM.all_models()["dense"]
    path = tmp_path / "w.qsf"
    offs = F.write_qsf(str(path), **kw)
    b = bytearray(path.read_bytes())
    b[offs["layer_offsets"][1] + 24 + 512 + 24 + 10] ^= 0x5A
    struct.pack_into("<Q", b, rc.layout["QSFHeader.total_file_size"], len(b) + 64)
    path.write_bytes(bytes(b))
    capfd.readouterr()
    got = rc.load(str(path))
    err = capfd.readouterr().err
    assert got["rc"] == 0
    assert "header CRC mismatch" in err and "file size mismatch" in err and "layer 1 CRC mismatch" in err
    struct.pack_into("<I", b, rc.layout["QSFHeader.magic"], 0x12345678)
    path.write_bytes(bytes(b))
    assert rc.load(str(path))["rc"] != 0
