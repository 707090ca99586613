"""The GPU path against the reference's own outputs (tests/golden/, written
by QStream's compiled quant.c/kernels_scalar.c)."""
from __future__ import annotations

import os

import numpy as np
import pytest

from tests.gpu_util import REL_L2, rel_l2

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "qsf_ref_vectors.npz")


@pytest.fixture(scope="module")
def kt():
    from qstream_amd import qsf_hip
    qsf_hip.init(0)
    return qsf_hip.KernelTable()


SLOT = {0: "matvec_2bit", 2: "matvec_3bit", 3: "matvec_4bit", 4: "matvec_4bit_sym",
        9: "matvec_outlier_2bit", 10: "matvec_outlier_4bit"}


def test_golden_matvecs(kt):
    g = np.load(GOLDEN, allow_pickle=False)
    worst = 0.0
    for name in g["mv_cases"]:
        qt, rows, cols, bs = (int(v) for v in g[name + "_meta"])
        out = np.full(rows, np.nan, np.float32)
        getattr(kt, SLOT[qt])(g[name + "_w"], g[name + "_x"], out, rows, cols, bs)
        err = rel_l2(out, g[name + "_y"])
        worst = max(worst, err)
        assert err <= REL_L2, (name, err)
    print(f"worst rel_l2 over {len(g['mv_cases'])} reference cases: {worst:.3e}")


def test_golden_ramp(kt):
    g = np.load(GOLDEN, allow_pickle=False)
    for qt, slot in ((3, kt.matvec_4bit), (0, kt.matvec_2bit)):
        out = np.zeros(4, np.float32)
        slot(g[f"ramp_q{qt}_w"], g[f"ramp_q{qt}_x"], out, 4, 64, 64)
        # the reference test's own bar (tests/test_core.c:635) and ours
        assert np.max(np.abs(out - g[f"ramp_q{qt}_y"])) <= 1e-3
        assert rel_l2(out, g[f"ramp_q{qt}_y"]) <= REL_L2
