"""QSF file -> device arena (qsf_hip_model_load) on the GPU: every tensor of
a small two-layer model file (blockwise matrices of several types and
per-tensor overrides, an outlier tensor, FP16 norms, embedding, final
norm, separate or tied output head) is reached by (layer, tensor type) and
checked against the oracle on the file's own bytes."""
from __future__ import annotations

import numpy as np
import pytest

from qstream_amd import qsf_format as F
from tests.gpu_util import REL_L2, dev, device_floats, host, rel_l2, torch_cuda

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    from qstream_amd import qsf_hip
    qsf_hip.init(0)
    return qsf_hip


def build(rng, tied, hidden=256, vocab=320, inter=512, bs=64):
    mk = lambda qt, r, c: F.quantize_matrix(F.heavy_tail_weights(rng, r, c) if qt == F.Q2_OUTLIER  # noqa
                                            else F.gaussian(rng, (r, c), 0.02), qt, bs)
    layers = []
    for li in range(2):
        recs = [(F.T_ATTN_NORM_W, F.FP16, 1, hidden, F.gaussian(rng, hidden).astype(np.float16).tobytes()),
                (F.T_ATTN_Q, 0xFF, hidden, hidden, mk(F.Q4, hidden, hidden)),   # layer default (4-bit)
                (F.T_ATTN_K, F.Q4SYM, hidden, hidden, mk(F.Q4SYM, hidden, hidden)),
                (F.T_FFN_GATE, F.Q2_OUTLIER, inter, hidden, mk(F.Q2_OUTLIER, inter, hidden)),
                (F.T_FFN_DOWN, F.Q3, hidden, inter, mk(F.Q3, hidden, inter)),
                (F.T_FFN_NORM_W, F.FP16, 1, hidden, F.gaussian(rng, hidden).astype(np.float16).tobytes())]
        layers.append(recs)
    emb = (F.Q4, mk(F.Q4, vocab, hidden))
    head = None if tied else mk(F.Q4, vocab, hidden)
    return dict(hidden=hidden, heads=4, kv_heads=2, vocab=vocab, inter=inter, layers=layers,
                quant_type=F.Q4, block_size=bs, embedding=emb,
                final_norm=F.gaussian(rng, hidden).astype(np.float16), output_head=head, tied=tied)


def check_model(hip, oracle, m, kw):
    torch = torch_cuda()
    info = m.info
    hidden, vocab, bs = kw["hidden"], kw["vocab"], kw["block_size"]
    assert (info.num_layers, info.hidden_dim, info.num_heads, info.num_kv_heads, info.vocab_size,
            info.head_dim, info.block_size) == (2, hidden, 4, 2, vocab, hidden // 4, bs)
    assert info.num_tensors == 12 and info.has_embedding == 1
    rng = np.random.default_rng(5)
    for li, recs in enumerate(kw["layers"]):
        for ttype, qt, rows, cols, payload in recs:
            if qt == F.FP16:
                p, n = m.vector(li, ttype)
                assert n == cols
                want = np.frombuffer(payload, np.float16).astype(np.float32)
                assert np.array_equal(device_floats(p, n), want)
                continue
            t = m.tensor(li, ttype)
            assert t is not None, (li, ttype)
            x = F.gaussian(rng, cols)
            y = torch.full((rows,), float("nan"), device="cuda:0")
            t.matvec(dev(x), y, stream=torch.cuda.current_stream())
            qeff = kw["quant_type"] if qt == 0xFF else qt
            ref = oracle.matvec(qeff, payload, x, rows, cols, bs)
            assert rel_l2(host(y), ref) <= REL_L2, (li, ttype, qt)
    assert m.tensor(0, F.T_ATTN_V) is None and m.vector(1, F.T_ATTN_Q)[0] is None
    # embedding rows, bit-exact
    eqt, epay = kw["embedding"]
    out = torch.empty(hidden, device="cuda:0")
    for token in (0, vocab - 1):
        hip.embed_row(m.embedding(), token, out, stream=torch.cuda.current_stream())
        assert np.array_equal(host(out), oracle.embed_row(eqt, epay, bs, hidden, token))
    # final norm and the logits matvec (src/engine.c:1190-1244)
    w, b = m.final_norm()
    assert b is None
    assert np.array_equal(device_floats(w, hidden),
                          np.asarray(kw["final_norm"], np.float16).astype(np.float32))
    x = F.gaussian(rng, hidden)
    y = torch.full((vocab,), float("nan"), device="cuda:0")
    m.output_head().matvec(dev(x), y, stream=torch.cuda.current_stream())
    head = epay if kw["tied"] else kw["output_head"]
    assert rel_l2(host(y), oracle.matvec(F.Q4, head, x, vocab, hidden, bs)) <= REL_L2


@pytest.mark.parametrize("tied", [False, True])
def test_model_load_every_tensor(hip, oracle, tmp_path, tied):
    kw = build(np.random.default_rng(7 + tied), tied)
    path = tmp_path / "m.qsf"
    F.write_qsf(str(path), **kw)
    m = hip.Model(str(path))
    assert m.info.crc_mismatches == 0 and m.info.size_mismatch == 0
    check_model(hip, oracle, m, kw)
    m.free()


def test_crc_mismatch_warns_and_loads_the_bytes(hip, oracle, tmp_path):
    """As the reference (src/format.c:226-233), a wrong layer CRC is counted
    and warned about, and the file's bytes are used as they are."""
    kw = build(np.random.default_rng(9), False)
    path = tmp_path / "c.qsf"
    offs = F.write_qsf(str(path), **kw, header_crc=False)
    b = bytearray(path.read_bytes())
    # flip a code byte inside layer 1's q payload (after norm record + q header + 4 meta bytes)
    pos = offs["layer_offsets"][1] + 24 + 512 + 24 + 4 + 10
    b[pos] ^= 0x5A
    path.write_bytes(bytes(b))
    rec = kw["layers"][1][1]
    pay = bytearray(rec[4])
    pay[4 + 10] ^= 0x5A
    kw["layers"][1][1] = rec[:4] + (bytes(pay),)
    m = hip.Model(str(path))
    assert m.info.crc_mismatches == 2            # the header (no CRC written) and layer 1
    check_model(hip, oracle, m, kw)
    m.free()


def test_fp16_embedding_rows_at_the_engine_stride(hip, tmp_path):
    """An FP16 table whose width is not a whole number of blocks: the
    engine reads token t at t * ceil(hd / bs) * bs * 2 bytes and converts hd
    values (src/engine.c:718-737, src/quant.c:82), so the file's rows are
    padded to whole blocks and the device table holds the first hd of
    each."""
    torch = torch_cuda()
    rng = np.random.default_rng(13)
    kw = build(rng, True)
    hidden, vocab, bs = 96, 260, 64
    q4 = lambda r, c: F.quantize_matrix(F.gaussian(rng, (r, c), 0.02), F.Q4, bs)  # noqa: E731
    kw.update(hidden=hidden, vocab=vocab, inter=128, heads=4, kv_heads=2, output_head=q4(vocab, hidden),
              tied=False, final_norm=F.gaussian(rng, hidden).astype(np.float16),
              layers=[[(F.T_ATTN_Q, F.Q4, hidden, hidden, q4(hidden, hidden))]])
    padded = F.gaussian(rng, (vocab, 128)).astype(np.float16)
    kw["embedding"] = (F.FP16, padded.tobytes())
    path = tmp_path / "f16.qsf"
    F.write_qsf(str(path), **kw)
    m = hip.Model(str(path))
    assert m.info.crc_mismatches == 0
    table = m.embedding_fp16()
    out = torch.empty(hidden, device="cuda:0")
    for token in (0, 1, vocab - 1):
        hip.embed_row_fp16(table, hidden, token, out, stream=torch.cuda.current_stream())
        assert np.array_equal(host(out), padded[token, :hidden].astype(np.float32))
    m.free()


def test_outlier_embedding_tied_head(hip, oracle, tmp_path):
    """A 2-bit + outlier model with a tied head, as the converter writes it
    (the embedding in the model's type, outlier table first,
    tools/convert_hf.py:206-208): its checked span is the whole table (no
    CRC warning), the tied logits are the outlier matvec over it
    (src/engine.c:1200-1226), and the row lookup, which the engine sizes as
    0 bytes for this type (src/engine.c:718-721), is refused."""
    torch = torch_cuda()
    rng = np.random.default_rng(17)
    kw = build(rng, True)
    hidden, vocab, bs = kw["hidden"], kw["vocab"], kw["block_size"]
    epay = F.quantize_matrix(F.heavy_tail_weights(rng, vocab, hidden), F.Q2_OUTLIER, bs)
    for recs in kw["layers"]:                    # the layer default is now type 9
        recs[:] = [r for r in recs if r[1] != 0xFF]
    kw.update(quant_type=F.Q2_OUTLIER, embedding=(F.Q2_OUTLIER, epay))
    path = tmp_path / "t9.qsf"
    F.write_qsf(str(path), **kw)
    m = hip.Model(str(path))
    assert m.info.crc_mismatches == 0 and m.info.size_mismatch == 0
    x = F.gaussian(rng, hidden)
    y = torch.full((vocab,), float("nan"), device="cuda:0")
    m.output_head().matvec(dev(x), y, stream=torch.cuda.current_stream())
    assert rel_l2(host(y), oracle.matvec(F.Q2_OUTLIER, epay, x, vocab, hidden, bs)) <= REL_L2
    out = torch.empty(hidden, device="cuda:0")
    with pytest.raises(hip.QsfHipError, match="no embedding lookup"):
        hip.embed_row(m.embedding(), 0, out, stream=torch.cuda.current_stream())
    m.free()


@pytest.mark.parametrize("name", ["dense", "dense_tied", "outlier_tied", "moe"])
def test_model_info_equals_reference_parse(hip, tmp_path, name):
    """What this build's loader reports equals what QStream's own reader
    (src/format.c:99-201, compiled into oracle/_ref) parses from the same
    file: header fields, its zero defaults resolved (src/format.c:145-162),
    tensor records per layer and no CRC or size warning in either."""
    from oracle.oracle import ref_container
    import struct
    from tests import container_models as CM
    rc = ref_container()
    if rc is None:
        pytest.skip("oracle/_ref not built")
    kw = CM.all_models()[name]
    path = tmp_path / f"{name}.qsf"
    F.write_qsf(str(path), **kw)
    ref = rc.load(str(path))
    assert ref["rc"] == 0
    L, hb = rc.layout, ref["header"]

    def h(f, t="I"):
        return struct.unpack_from("<" + t, hb, L[f"QSFHeader.{f}"])[0]

    m = hip.Model(str(path))
    try:
        i = m.info
        assert (i.num_layers, i.hidden_dim, i.num_heads, i.vocab_size, i.max_seq_len, i.intermediate_dim,
                i.block_size) == (h("num_layers"), h("hidden_dim"), h("num_heads"), h("vocab_size"),
                                  h("max_seq_len"), h("intermediate_dim"), h("block_size"))
        assert (i.num_kv_heads, i.head_dim, i.weight_tied) == (ref["num_kv_heads"], ref["head_dim"],
                                                               ref["weight_tied"])
        assert (i.quant_type, i.activation, i.norm_type, i.pos_enc_type, i.ffn_type, i.attn_type, i.has_bias) == \
            (h("quant_type", "B"), h("activation", "B"), h("norm_type", "B"), h("pos_enc_type", "B"),
             h("ffn_type", "B"), h("attn_type", "B"), h("has_bias", "B"))
        assert (i.num_experts, i.num_active_experts, i.moe_norm_topk, i.expert_intermediate_dim) == \
            (h("num_experts", "B"), h("num_active_experts", "B"), h("moe_norm_topk", "B"),
             h("expert_intermediate_dim"))
        assert (i.rope_theta, i.norm_epsilon) == (h("rope_theta", "f"), h("norm_epsilon", "f"))
        n_rec = sum(struct.unpack_from("<H", ref["layer_index"], k * L["QSFLayerIndex"] +
                                       L["QSFLayerIndex.num_tensors"])[0] for k in range(i.num_layers))
        assert i.num_tensors == n_rec
        assert i.crc_mismatches == 0 and i.size_mismatch == 0 and i.has_embedding == 1
        assert i.moe_layers == (i.num_layers if name == "moe" else 0)
    finally:
        m.free()
