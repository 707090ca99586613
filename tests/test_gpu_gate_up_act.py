"""The fused gate/up GEMV with the activation product (qsf_hip_gate_up_act_dev
over a qsf_hip_tensor_upload_pair tensor), through the C ABI.

  * Against the separate path (grouped gate/up GEMV, then qsf_hip_act_mul_dev)
    bit for bit where both launches take the same row-group width (rows of
    64 or more blocks: every row group is the whole wave either way).
  * Against the oracle (src/kernels_scalar.c matvecs, then the
    src/engine.c:1128-1140 activation product) to rel-L2 <= 1e-5 on every
    shape, ragged ones included.
  * Outlier formats are refused at upload.
"""
from __future__ import annotations

import numpy as np
import pytest

from qstream_amd import qsf_format as F
from tests.gpu_util import ENGINES, REL_L2, dev, engine_hip, host, rel_l2, torch_cuda

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", params=ENGINES, ids=lambda e: f"engine{e}")
def hip(request):
    yield from engine_hip(request)


# (qt, bs, rows, cols, same row groups as the separate path)
SHAPES = [
    (F.Q3, 128, 11008, 4096, True),    # the 7B FFN at 3-bit (the layer step's launch)
    (F.Q4, 64, 1024, 4096, True),
    (F.Q2, 256, 700, 16384, True),
    (F.Q4SYM, 32, 640, 2048, True),
    (F.Q4, 64, 300, 1000, False),      # ragged: 16 blocks a row, a partial last block
    (F.Q3, 64, 129, 200, False),
    (F.Q2, 128, 33, 130, False),
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"qt{s[0]}_bs{s[1]}_{s[2]}x{s[3]}")
def test_gate_up_act(hip, oracle, shape):
    qt, bs, rows, cols, same = shape
    torch = torch_cuda()
    rng = np.random.default_rng(rows + cols)
    pg = np.frombuffer(F.quantize_matrix(F.gaussian(rng, (rows, cols), 0.02), qt, bs), np.uint8).copy()
    pu = np.frombuffer(F.quantize_matrix(F.gaussian(rng, (rows, cols), 0.02), qt, bs), np.uint8).copy()
    x = F.gaussian(rng, cols)
    tg, tu = hip.Tensor(pg, qt, rows, cols, bs), hip.Tensor(pu, qt, rows, cols, bs)
    pair = hip.TensorPair(pg, pu, qt, rows, cols, bs)
    g_ref = oracle.matvec(qt, pg.tobytes(), x, rows, cols, bs)
    u_ref = oracle.matvec(qt, pu.tobytes(), x, rows, cols, bs)
    dx = dev(x)
    try:
        for act in (0, 1, 2, 3):
            print(f"gate_up_act qt {qt} bs {bs} {rows}x{cols} act {act}", flush=True)
            out = torch.full((rows,), float("nan"), device="cuda:0")
            pair.gate_up_act(dx, out, act)
            got = host(out)
            ref = oracle.vec_mul(oracle.act(act, g_ref), u_ref)
            assert rel_l2(got, ref) <= REL_L2, (act, rel_l2(got, ref))
            if same:
                g = torch.empty(rows, device="cuda:0")
                u = torch.empty(rows, device="cuda:0")
                hip.matvec_group([tg, tu], dx, [g, u])
                hip.act_mul(g, u, act)
                assert np.array_equal(host(g).view(np.uint32), got.view(np.uint32)), act
    finally:
        for t in (tg, tu, pair):
            t.free()


def test_pair_refuses_outlier_formats(hip):
    rng = np.random.default_rng(3)
    w = F.heavy_tail_weights(rng, 64, 256)
    p = np.frombuffer(F.quantize_matrix(w, F.Q2_OUTLIER, 64), np.uint8).copy()
    with pytest.raises(hip.QsfHipError):
        hip.TensorPair(p, p, F.Q2_OUTLIER, 64, 256, 64)
