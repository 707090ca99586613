"""The residual + NaN check + RMS norm fused into the matvec that consumes
the norm (qsf_hip_residual_norm_matvec_group_dev and
qsf_hip_residual_norm_gate_up_act_dev), through the C ABI.

  * Against the separate launches (qsf_hip_residual_norm_dev, then
    qsf_hip_matvec_group_dev / qsf_hip_gate_up_act_dev) bit for bit: the
    residual, the NaN-check index and every output row.  Both paths run the
    same norm arithmetic (src/engine.c:1174-1187, 940-948) and the same
    matvec kernel on the same x.
  * Against the oracle (the norm, then src/kernels_scalar.c matvecs) to
    rel-L2 <= 1e-5.
  * Refusals: outlier formats, an aliased residual, rows wider than 8192.
"""
from __future__ import annotations

import numpy as np
import pytest

from qstream_amd import qsf_format as F
from tests.gpu_util import ENGINES, REL_L2, dev, engine_hip, host, rel_l2, torch_cuda

pytestmark = pytest.mark.gpu

EPS = 1e-5


@pytest.fixture(scope="module", params=ENGINES, ids=lambda e: f"engine{e}")
def hip(request):
    yield from engine_hip(request)


def _vectors(rng, cols, poison):
    res = F.gaussian(rng, cols)
    x = F.gaussian(rng, cols)
    if poison == "nan":
        x[cols // 3] = np.nan
    elif poison == "big":
        x[7] = 3e30                       # finite, past the 1e30 check
    elif poison == "res_nan":
        res[cols // 2] = np.nan           # in the residual, not the increment
    w = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    return res, x, w


def _bits(a):
    return host(a).view(np.uint32)


def _bad_index(poison, cols):
    """First element the residual check flags (src/engine.c:1174-1187): -1,
    or the poisoned one."""
    return {None: -1, "nan": cols // 3, "big": 7, "res_nan": cols // 2}[poison]


# (qt, bs, [rows...], cols): q/k/v-like groups and single matrices, split
# views (block 128/256) and whole blocks, ragged widths
GROUPS = [
    (F.Q3, 128, [4096, 1024, 1024], 4096),
    (F.Q4, 64, [1000], 3000),
    (F.Q2, 256, [700, 33], 5000),
    (F.Q4SYM, 32, [300], 2048),
    (F.Q3, 64, [129], 200),
    (F.Q4, 128, [257], 8192),
]


@pytest.mark.parametrize("poison", [None, "nan", "big", "res_nan"])
@pytest.mark.parametrize("shape", GROUPS, ids=lambda s: f"qt{s[0]}_bs{s[1]}_{'-'.join(map(str, s[2]))}x{s[3]}")
def test_fused_group_equals_separate(hip, oracle, shape, poison):
    qt, bs, rows_list, cols = shape
    torch = torch_cuda()
    rng = np.random.default_rng(cols + len(rows_list))
    payloads = [np.frombuffer(F.quantize_matrix(F.gaussian(rng, (r, cols), 0.02), qt, bs), np.uint8).copy()
                for r in rows_list]
    ts = [hip.Tensor(p, qt, r, cols, bs) for p, r in zip(payloads, rows_list)]
    res, x, w = _vectors(rng, cols, poison)
    print(f"fused group qt {qt} bs {bs} rows {rows_list} cols {cols} poison {poison}", flush=True)
    try:
        # separate: residual + norm in place, then the group matvec
        r1 = dev(res)
        n1 = torch.empty(cols, device="cuda:0")
        bad1 = torch.full((1,), 7, dtype=torch.int32, device="cuda:0")
        hip.residual_norm(r1, dev(x), dev(w), EPS, n1, bad=bad1)
        y1 = [torch.full((r,), float("nan"), device="cuda:0") for r in rows_list]
        hip.matvec_group(ts, n1, y1)
        # fused
        r_in = dev(res)
        r2 = torch.full((cols,), float("nan"), device="cuda:0")
        bad2 = torch.full((1,), 7, dtype=torch.int32, device="cuda:0")
        y2 = [torch.full((r,), float("nan"), device="cuda:0") for r in rows_list]
        hip.residual_norm_matvec_group(ts, r_in, r2, dev(x), dev(w), EPS, y2, bad=bad2)
        assert np.array_equal(_bits(r1), _bits(r2))
        assert np.array_equal(_bits(r_in), res.view(np.uint32))   # the input residual is untouched
        assert int(host(bad1)[0]) == int(host(bad2)[0]) == _bad_index(poison, cols)
        for a, b in zip(y1, y2):
            assert np.array_equal(_bits(a), _bits(b))
        if poison is None:
            r = (res + x).astype(np.float32)
            nv = oracle.rms_norm(r, w, EPS)
            for p, rr, y in zip(payloads, rows_list, y2):
                ref = oracle.matvec(qt, p.tobytes(), nv, rr, cols, bs)
                assert rel_l2(host(y), ref) <= REL_L2
    finally:
        for t in ts:
            t.free()


@pytest.mark.parametrize("poison", [None, "nan", "big", "res_nan"])
@pytest.mark.parametrize("shape", [(F.Q3, 128, 11008, 4096), (F.Q4, 64, 300, 1000), (F.Q2, 256, 64, 2048)],
                         ids=lambda s: f"qt{s[0]}_bs{s[1]}_{s[2]}x{s[3]}")
def test_fused_gate_up_act_equals_separate(hip, oracle, shape, poison):
    qt, bs, rows, cols = shape
    torch = torch_cuda()
    rng = np.random.default_rng(rows)
    pg = np.frombuffer(F.quantize_matrix(F.gaussian(rng, (rows, cols), 0.02), qt, bs), np.uint8).copy()
    pu = np.frombuffer(F.quantize_matrix(F.gaussian(rng, (rows, cols), 0.02), qt, bs), np.uint8).copy()
    pair = hip.TensorPair(pg, pu, qt, rows, cols, bs)
    res, x, w = _vectors(rng, cols, poison)
    try:
        for act in (0, 2):
            print(f"fused gate/up qt {qt} bs {bs} {rows}x{cols} act {act} poison {poison}", flush=True)
            r1 = dev(res)
            n1 = torch.empty(cols, device="cuda:0")
            bad1 = torch.full((1,), 7, dtype=torch.int32, device="cuda:0")
            hip.residual_norm(r1, dev(x), dev(w), EPS, n1, bad=bad1)
            o1 = torch.full((rows,), float("nan"), device="cuda:0")
            pair.gate_up_act(n1, o1, act)
            r2 = torch.full((cols,), float("nan"), device="cuda:0")
            o2 = torch.full((rows,), float("nan"), device="cuda:0")
            bad = torch.full((1,), 7, dtype=torch.int32, device="cuda:0")
            pair.residual_norm_gate_up_act(dev(res), r2, dev(x), dev(w), EPS, o2, act, bad=bad)
            assert np.array_equal(_bits(r1), _bits(r2))
            assert np.array_equal(_bits(o1), _bits(o2))
            assert int(host(bad)[0]) == int(host(bad1)[0]) == _bad_index(poison, cols)
            if poison is not None:
                continue
            nv = oracle.rms_norm((res + x).astype(np.float32), w, EPS)
            g = oracle.matvec(qt, pg.tobytes(), nv, rows, cols, bs)
            u = oracle.matvec(qt, pu.tobytes(), nv, rows, cols, bs)
            assert rel_l2(host(o2), oracle.vec_mul(oracle.act(act, g), u)) <= REL_L2
    finally:
        pair.free()


def test_fused_refusals(hip):
    torch = torch_cuda()
    rng = np.random.default_rng(5)
    cols = 256
    res, x, w = _vectors(rng, cols, None)
    po = np.frombuffer(F.quantize_matrix(F.heavy_tail_weights(rng, 64, cols), F.Q2_OUTLIER, 64),
                       np.uint8).copy()
    pp = np.frombuffer(F.quantize_matrix(F.gaussian(rng, (64, cols), 0.02), F.Q4, 64), np.uint8).copy()
    pw = np.frombuffer(F.quantize_matrix(F.gaussian(rng, (8, 8200), 0.02), F.Q4, 64), np.uint8).copy()
    to, tp, tw = (hip.Tensor(po, F.Q2_OUTLIER, 64, cols, 64), hip.Tensor(pp, F.Q4, 64, cols, 64),
                  hip.Tensor(pw, F.Q4, 8, 8200, 64))
    try:
        r, r2, dx, dw = dev(res), torch.empty(cols, device="cuda:0"), dev(x), dev(w)
        y = torch.empty(64, device="cuda:0")
        with pytest.raises(hip.QsfHipError):
            hip.residual_norm_matvec_group([to], r, r2, dx, dw, EPS, [y])          # outliers
        with pytest.raises(hip.QsfHipError):
            hip.residual_norm_matvec_group([tp], r, r, dx, dw, EPS, [y])           # res_out == res
        with pytest.raises(hip.QsfHipError):
            hip.residual_norm_matvec_group([tp], r, r2, dx, dw, EPS, [r2])         # y == res_out
        wide = torch.zeros(8200, device="cuda:0")
        with pytest.raises(hip.QsfHipError):
            hip.residual_norm_matvec_group([tw], wide, torch.empty(8200, device="cuda:0"), wide.clone(),
                                           torch.ones(8200, device="cuda:0"), EPS,
                                           [torch.empty(8, device="cuda:0")])  # cols > 8192
        assert np.array_equal(host(r), res)
    finally:
        for t in (to, tp, tw):
            t.free()
