"""GPT-OSS MXFP4 checkpoint tensors -> QSF file (convert_mxfp4) -> device
arena (qsf_hip_model_load) on the GPU: each expert's gate, up and down
reproduce GPT-OSS's gate_up[::2] / gate_up[1::2] / down products on the
checkpoint's codes, and the layer's MoE table (built at load with its FP16
biases) runs router logits -> top-k -> experts like the oracle."""
from __future__ import annotations

import numpy as np
import pytest

from qstream_amd import convert_mxfp4 as M
from qstream_amd import qsf_format as F
from tests.gpu_util import REL_L2, dev, host, rel_l2, torch_cuda
from tests.test_convert_mxfp4 import gpt_oss_layer

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    from qstream_amd import qsf_hip
    qsf_hip.init(0)
    return qsf_hip


@pytest.mark.parametrize("bias", [True, False])
def test_converted_gpt_oss_layer_runs(hip, oracle, tmp_path, bias):
    torch = torch_cuda()
    s = torch.cuda.current_stream()
    rng = np.random.default_rng(31 + bias)
    n_exp, hidden, inter, k = 4, 256, 128, 2
    t = gpt_oss_layer(rng, n_exp, hidden, inter, bias=bias)
    recs = M.moe_layer_records(t, 0)
    path = tmp_path / "gptoss.qsf"
    F.write_qsf(str(path), hidden=hidden, heads=4, vocab=128, inter=inter, layers=[recs],
                quant_type=F.Q4, ffn_type=F.FFN_MOE, num_experts=n_exp, num_active_experts=k,
                moe_norm_topk=1, expert_dim=inter)
    m = hip.Model(str(path))
    info = m.info
    assert (info.num_experts, info.num_active_experts, info.moe_norm_topk,
            info.expert_intermediate_dim, info.moe_layers) == (n_exp, k, 1, inter, 1)

    p = "model.layers.0.mlp.experts."
    x = F.gaussian(rng, hidden)
    for e in range(n_exp):
        gate_up = M.dequant_mxfp4(t[p + "gate_up_proj_blocks"][e],
                                  t[p + "gate_up_proj_scales"][e]).astype(np.float64) @ x
        y = torch.full((inter,), float("nan"), device="cuda:0")
        m.tensor(0, F.t_moe(e, "gate")).matvec(dev(x), y, stream=s)
        assert rel_l2(host(y), gate_up[0::2]) <= REL_L2
        m.tensor(0, F.t_moe(e, "up")).matvec(dev(x), y, stream=s)
        assert rel_l2(host(y), gate_up[1::2]) <= REL_L2
        xi = F.gaussian(rng, inter)
        down = M.dequant_mxfp4(t[p + "down_proj_blocks"][e],
                               t[p + "down_proj_scales"][e]).astype(np.float64) @ xi
        yd = torch.full((hidden,), float("nan"), device="cuda:0")
        m.tensor(0, F.t_moe(e, "down")).matvec(dev(xi), yd, stream=s)
        assert rel_l2(host(yd), down) <= REL_L2

    # router -> MoE (src/engine.c:968-1107); logits from the layer's router tensor
    by_type = {r[0]: r for r in recs}
    _, rqt, _, _, rpay = by_type[F.T_MOE_ROUTER]
    logits = torch.full((n_exp,), float("nan"), device="cuda:0")
    m.tensor(0, F.T_MOE_ROUTER).matvec(dev(x), logits, stream=s)
    ref_logits = oracle.matvec(rqt, rpay, x, n_exp, hidden, 64)
    assert rel_l2(host(logits), ref_logits) <= REL_L2
    ex = []
    for e in range(n_exp):
        d = {role: by_type[F.t_moe(e, role)][4] for role in ("gate", "up", "down")}
        if bias:
            for role in ("gate", "up", "down"):
                d[role + "_bias"] = np.frombuffer(by_type[F.t_moe(e, role, True)][4], np.uint16)
        ex.append(d)
    for act in (2, 0):
        ref = oracle.moe_token(ex, k, 1, act, hidden, inter, x, ref_logits)
        out = torch.full((1, hidden), float("nan"), device="cuda:0")
        m.moe(0).forward(k, 1, act, 1, dev(x), dev(ref_logits), out, stream=s)
        assert rel_l2(host(out)[0], ref) <= REL_L2, act
    m.free()


def test_dense_experts_get_no_moe_table(hip, tmp_path):
    """Experts re-quantised to a block type (the reference converter's
    only path) load as ordinary tensors; no MXFP4 table is built."""
    rng = np.random.default_rng(40)
    t = gpt_oss_layer(rng, 2, 128, 64, bias=False)
    recs = M.moe_layer_records(t, 0, quant=F.Q4, block_size=64)
    path = tmp_path / "dense.qsf"
    F.write_qsf(str(path), hidden=128, heads=4, vocab=128, inter=64, layers=[recs],
                quant_type=F.Q4, ffn_type=F.FFN_MOE, num_experts=2, num_active_experts=1,
                expert_dim=64)
    m = hip.Model(str(path))
    assert m.info.moe_layers == 0 and m.moe(0) is None
    assert m.tensor(0, F.t_moe(1, "down")) is not None
    m.free()
