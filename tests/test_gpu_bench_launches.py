"""The exact launches bench.py times, on the benchmark's own seeded data
(qsf_format.config*), against the oracle at the 1e-5 rel-L2 bar:

* config 0: one 4-bit 4096x4096 launch;
* config 1: gate and up (2-bit+outlier 11008x4096) grouped in one launch;
* config 2: one 3-bit 7B layer as bench_layers launches it -- q/k/v grouped
  (n=3, 4096x4096), o alone, gate/up grouped (n=2, 11008x4096), down alone
  (4096x11008), each on its own x.

A grouped launch must equal the same matrices' single launches bit for
bit: grouping changes the grid, not the arithmetic of a row.
"""
from __future__ import annotations

import numpy as np
import pytest

from qstream_amd import qsf_format as F
from tests.gpu_util import REL_L2, dev, host, rel_l2, torch_cuda

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    from qstream_amd import qsf_hip
    qsf_hip.init(0)
    return qsf_hip


@pytest.fixture(scope="module")
def layer():
    return F.config2_layer()


def _launch(hip, tensors, x, rows):
    torch = torch_cuda()
    ys = [torch.full((r,), float("nan"), device="cuda:0") for r in rows]
    hip.matvec_group(tensors, dev(x), ys, stream=torch.cuda.current_stream())
    return [host(y) for y in ys]


def _check_group(hip, oracle, qt, bs, mats, x, label):
    tens = [hip.Tensor(p, qt, r, c, bs) for _, p, r, c in mats]
    rows = [r for _, _, r, _ in mats]
    grouped = _launch(hip, tens, x, rows)
    for t, (name, p, r, c), got in zip(tens, mats, grouped):
        single = _launch(hip, [t], x, [r])[0]
        ref = oracle.matvec(qt, p, x, r, c, bs)
        err = rel_l2(got, ref)
        print(f"{label} {name} {r}x{c}: rel_l2 {err:.3e}")
        assert np.array_equal(got, single), f"{name}: grouped launch differs from its single launch"
        assert err <= REL_L2, (name, err)
    for t in tens:
        t.free()


def test_config0_launch(hip, oracle):
    qt, bs, mats, x = F.config0_matrix()
    _check_group(hip, oracle, qt, bs, mats, x, "cfg0")


def test_config1_gate_up_grouped(hip, oracle):
    qt, bs, mats, x = F.config1_matrices()
    _check_group(hip, oracle, qt, bs, mats, x, "cfg1")


@pytest.mark.parametrize("names", [("q", "k", "v"), ("o",), ("gate", "up"), ("down",)])
def test_config2_layer_launches(hip, oracle, layer, names):
    qt, bs, mats = layer
    sel = [m for m in mats if m[0] in names]
    rng = np.random.default_rng(20 + len(names) * 7 + sel[0][3])
    x = F.gaussian(rng, sel[0][3])
    _check_group(hip, oracle, qt, bs, sel, x, "cfg2")
