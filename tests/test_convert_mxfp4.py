"""GPT-OSS MXFP4 -> QSF converter (qstream_amd.convert_mxfp4): scale
semantics, element order, gate/up split and the written records, checked
against the oracle's MXFP4 matvec and fp64 arithmetic on the checkpoint's
own codes."""
from __future__ import annotations

import math
import struct

import numpy as np
import pytest

from qstream_amd import convert_mxfp4 as M
from qstream_amd import qsf_format as F


def gpt_oss_layer(rng, n_exp=3, hidden=128, inter=64, bias=True, layer=0):
    """A GPT-OSS-shaped MoE block with MXFP4 codes of N(0, 0.02) weights."""
    def packed(rows, cols):
        p = np.frombuffer(F.quantize_mxfp4(F.gaussian(rng, (rows, cols), 0.02)), np.uint8)
        nb = cols // 32
        return p[:rows * nb * 16].reshape(rows, nb, 16), p[rows * nb * 16:].reshape(rows, nb)
    # bf16-representable values, as the checkpoint's bf16 tensors widen
    bf = lambda a: (a.view(np.uint32) & 0xFFFF0000).view(np.float32)  # noqa: E731
    gu = [packed(2 * inter, hidden) for _ in range(n_exp)]
    dn = [packed(hidden, inter) for _ in range(n_exp)]
    p = f"model.layers.{layer}.mlp"
    t = {f"{p}.experts.gate_up_proj_blocks": np.stack([b for b, _ in gu]),
         f"{p}.experts.gate_up_proj_scales": np.stack([s for _, s in gu]),
         f"{p}.experts.down_proj_blocks": np.stack([b for b, _ in dn]),
         f"{p}.experts.down_proj_scales": np.stack([s for _, s in dn]),
         f"{p}.router.weight": bf(F.gaussian(rng, (n_exp, hidden), 0.02))}
    if bias:
        t[f"{p}.experts.gate_up_proj_bias"] = bf(F.gaussian(rng, (n_exp, 2 * inter), 0.05))
        t[f"{p}.experts.down_proj_bias"] = bf(F.gaussian(rng, (n_exp, hidden), 0.05))
        t[f"{p}.router.bias"] = bf(F.gaussian(rng, n_exp, 0.1))
    return t


def test_e8m0_scale_is_a_power_of_two_and_255_is_nan():
    """OCP MX v1.0: E8M0 byte E encodes 2^(E-127); 255 is NaN.  The
    reference converter multiplies by the byte itself (E=127 -> x127)."""
    e = np.arange(255, dtype=np.uint8)
    got = M.e8m0_scale(e).astype(np.float64)
    assert np.array_equal(got, [math.ldexp(1.0, int(v) - 127) for v in e])
    assert np.isnan(M.e8m0_scale(np.uint8(255)))
    assert M.e8m0_scale(np.uint8(127)) == 1.0 and M.e8m0_scale(np.uint8(0)) == 2.0 ** -127


def test_dequant_matches_the_oracle_decode(oracle):
    """Every code x a spread of scales: dequant_mxfp4 equals the oracle's
    E2M1 decode times the scale, and the low nibble is element 2j."""
    codes = np.arange(256, dtype=np.uint8)            # every (lo, hi) pair
    blocks = np.resize(codes, (16, 16)).reshape(1, 16, 16)
    scales = np.array([[0, 1, 64, 100, 126, 127, 128, 130, 150, 200, 230, 250, 252, 253, 254, 120]],
                      np.uint8)
    with np.errstate(over="ignore"):                  # 6 * 2^127 is +Inf in fp32
        got = M.dequant_mxfp4(blocks, scales)[0].reshape(16, 32)
    for b in range(16):
        s = math.ldexp(1.0, int(scales[0, b]) - 127)
        for j in range(16):
            byte = int(blocks[0, b, j])
            for k, nib in ((0, byte & 15), (1, byte >> 4)):
                want = np.float32(oracle.lib.orc_e2m1_to_fp32(nib)) * np.float64(s)
                with np.errstate(over="ignore"):
                    assert got[b, 2 * j + k] == np.float32(want), (b, j, k)


def test_payload_matvec_equals_fp64_dequant(oracle):
    """The written payload, run through the oracle's MXFP4 matvec, gives
    W x with W the checkpoint's dequantised codes (fp64 reference)."""
    rng = np.random.default_rng(1)
    t = gpt_oss_layer(rng, n_exp=1, hidden=256, inter=96, bias=False)
    b = t["model.layers.0.mlp.experts.down_proj_blocks"][0]
    s = t["model.layers.0.mlp.experts.down_proj_scales"][0]
    x = F.gaussian(rng, 96)
    w = M.dequant_mxfp4(b, s).astype(np.float64)
    got = oracle.matvec(F.MXFP4, M.mxfp4_payload(b, s), x, 256, 96, 32)
    want = w @ x.astype(np.float64)
    assert np.max(np.abs(got - want)) <= 1e-6 * np.max(np.abs(want))


def test_payload_round_trips_the_test_writer():
    rng = np.random.default_rng(2)
    w = F.gaussian(rng, (40, 160), 0.02)
    p = np.frombuffer(F.quantize_mxfp4(w), np.uint8)
    b, s = p[:40 * 5 * 16].reshape(40, 5, 16), p[40 * 5 * 16:].reshape(40, 5)
    assert M.mxfp4_payload(b, s) == p.tobytes()
    with pytest.raises(ValueError):
        M.mxfp4_payload(b[:, :, :8], s)


def test_gate_up_split_follows_gpt_oss():
    """GPT-OSS takes gate_up[..., ::2] as gate and [..., 1::2] as up of
    gate_up = x W^T + b: the even and odd output rows.  The interleaved
    split reproduces that; the reference's halves split does not."""
    rng = np.random.default_rng(3)
    t = gpt_oss_layer(rng, n_exp=2, hidden=128, inter=64)
    p = "model.layers.0.mlp.experts."
    blocks, scales = t[p + "gate_up_proj_blocks"], t[p + "gate_up_proj_scales"]
    bias = t[p + "gate_up_proj_bias"]
    x = F.gaussian(rng, 128).astype(np.float64)
    for e in range(2):
        gate_up = M.dequant_mxfp4(blocks[e], scales[e]).astype(np.float64) @ x + bias[e]
        (gb, ub), (gs, us) = M.split_gate_up(blocks, "interleave"), M.split_gate_up(scales, "interleave")
        g_bias, u_bias = M.split_gate_up(bias, "interleave")
        gate = M.dequant_mxfp4(gb[e], gs[e]).astype(np.float64) @ x + g_bias[e]
        up = M.dequant_mxfp4(ub[e], us[e]).astype(np.float64) @ x + u_bias[e]
        assert np.array_equal(gate, gate_up[0::2]) and np.array_equal(up, gate_up[1::2])
        (hb, _), (hs, _) = M.split_gate_up(blocks, "halves"), M.split_gate_up(scales, "halves")
        halves_gate = M.dequant_mxfp4(hb[e], hs[e]).astype(np.float64) @ x
        assert not np.allclose(halves_gate + g_bias[e], gate_up[0::2])
    with pytest.raises(ValueError):
        M.split_gate_up(blocks, "sideways")


@pytest.mark.parametrize("split", ["interleave", "halves"])
def test_layer_records(oracle, split):
    rng = np.random.default_rng(4)
    n_exp, hidden, inter = 3, 128, 64
    t = gpt_oss_layer(rng, n_exp, hidden, inter)
    recs = M.moe_layer_records(t, 0, split=split)
    by_type = {r[0]: r for r in recs}
    assert len(recs) == len(by_type) == 2 + 6 * n_exp
    rt, rqt, rr, rc, rpay = by_type[F.T_MOE_ROUTER]
    assert (rqt, rr, rc) == (F.Q4, n_exp, hidden)
    p = "model.layers.0.mlp.experts."
    (gb, ub), (gs, us) = (M.split_gate_up(t[p + "gate_up_proj_blocks"], split),
                          M.split_gate_up(t[p + "gate_up_proj_scales"], split))
    g_bias, u_bias = M.split_gate_up(t[p + "gate_up_proj_bias"], split)
    for e in range(n_exp):
        for role, b, s, rows, cols in (("gate", gb, gs, inter, hidden), ("up", ub, us, inter, hidden),
                                       ("down", t[p + "down_proj_blocks"], t[p + "down_proj_scales"],
                                        hidden, inter)):
            _, qt, r, c, pay = by_type[F.t_moe(e, role)]
            assert (qt, r, c) == (F.MXFP4, rows, cols)
            assert pay == M.mxfp4_payload(b[e], s[e])        # the checkpoint's bytes
        for role, v in (("gate", g_bias[e]), ("up", u_bias[e]), ("down", t[p + "down_proj_bias"][e])):
            _, qt, r, c, pay = by_type[F.t_moe(e, role, True)]
            assert (qt, r, c) == (F.FP16, 1, v.size)
            assert np.array_equal(np.frombuffer(pay, np.float16), v.astype(np.float16))


def test_requantised_experts_use_the_fixed_scale(oracle):
    """quant != MXFP4: the experts are dequantised with 2^(E-127) and
    quantised again to the block type, as the reference converter does
    (with its raw-byte scale fixed)."""
    rng = np.random.default_rng(5)
    t = gpt_oss_layer(rng, n_exp=1, hidden=128, inter=64, bias=False)
    recs = {r[0]: r for r in M.moe_layer_records(t, 0, quant=F.Q4, block_size=32)}
    _, qt, rows, cols, pay = recs[F.t_moe(0, "down")]
    assert (qt, rows, cols) == (F.Q4, 128, 64)
    p = "model.layers.0.mlp.experts."
    w = M.dequant_mxfp4(t[p + "down_proj_blocks"][0], t[p + "down_proj_scales"][0])
    assert pay == F.quantize_matrix(w, F.Q4, 32)
    x = F.gaussian(rng, 64)
    got = oracle.matvec(F.Q4, pay, x, 128, 64, 32)
    want = w.astype(np.float64) @ x
    assert np.linalg.norm(got - want) <= 0.1 * np.linalg.norm(want)   # 4-bit re-quantisation


def test_safetensors_layer_and_moe_header(tmp_path):
    torch = pytest.importorskip("torch")
    st = pytest.importorskip("safetensors.torch")
    rng = np.random.default_rng(6)
    t = gpt_oss_layer(rng, n_exp=2, hidden=64, inter=32, layer=3)
    tt = {k: (torch.from_numpy(v).to(torch.bfloat16) if v.dtype == np.float32 else torch.from_numpy(v))
          for k, v in t.items()}
    tt["model.layers.3.self_attn.q_proj.weight"] = torch.zeros(4, 4)
    path = str(tmp_path / "layer.safetensors")
    st.save_file(tt, path)
    got = M.load_gpt_oss_layer(path, 3)
    assert set(got) == set(t)
    for k, v in t.items():
        assert got[k].dtype == v.dtype and np.array_equal(got[k], v), k
    recs = M.moe_layer_records(got, 3)
    q = tmp_path / "m.qsf"
    F.write_qsf(str(q), hidden=64, heads=4, vocab=128, inter=32, layers=[recs], quant_type=F.Q4,
                ffn_type=F.FFN_MOE, num_experts=2, num_active_experts=2, moe_norm_topk=1,
                expert_dim=32)
    h = q.read_bytes()[:256]
    assert struct.unpack_from("<BBBBI", h, 173) == (2, 2, 1, 0, 32) and h[141] == F.FFN_MOE
    import zlib
    assert struct.unpack_from("<I", h, 168)[0] == zlib.crc32(h[:168]) & 0xFFFFFFFF
