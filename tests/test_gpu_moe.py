"""GPU parity of the MXFP4 matvec and the MoE FFN against the CPU oracle.

The oracle restates src/engine.c:951-1107 (softmax, strict '>' top-K,
renormalisation, gate/up/act/mul/down, rank-order weighted sum) with the
MXFP4 element order of tools/convert_hf.py:1456-1495 and the OCP MX scale.
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


def _stream():
    return torch_cuda().cuda.current_stream()


def test_mxfp4_unpack_every_code_and_scale(hip, oracle):
    """All 16 E2M1 codes in both nibble positions x a sweep of E8M0 scales,
    through the table slot with one-hot activations: output row r, input
    col c gives exactly e2m1(code) * 2^(E-127).  The ends of the scale
    range are OCP MX's special cases: E = 0 is 2^-127 (an fp32 subnormal,
    kept, not flushed) and E = 255 is NaN, which every product carries,
    code 0 included."""
    rows, cols = 16, 32
    codes = np.zeros((rows, 1, 16), np.uint8)
    for r in range(rows):
        for j in range(16):
            lo, hi = (r + 2 * j) % 16, (r + 2 * j + 1) % 16
            codes[r, 0, j] = lo | (hi << 4)
    kt = hip.KernelTable()
    for e in (0, 1, 100, 127, 130, 200, 254, 255):
        scales = np.full((rows, 1), e, np.uint8)
        payload = codes.tobytes() + scales.tobytes()
        got = np.zeros((cols, rows), np.float32)
        for c in range(cols):
            x = np.zeros(cols, np.float32)
            x[c] = 1.0
            kt.matvec_mxfp4(payload, x, got[c], rows, cols, 32)
        for r in range(rows):
            for c in range(cols):
                nib = (codes[r, 0, c // 2] >> (4 * (c % 2))) & 15
                if e == 255:
                    assert np.isnan(got[c, r]), (e, r, c, got[c, r])
                    continue
                want = np.float32(oracle.lib.orc_e2m1_to_fp32(int(nib))) * np.float32(2.0 ** (e - 127))
                assert got[c, r] == want, (e, r, c, got[c, r], want)


@pytest.mark.parametrize("rows,cols", [(64, 64), (2880, 2880), (100, 320), (7, 96)])
def test_mxfp4_matvec(hip, oracle, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    w = F.gaussian(rng, (rows, cols), 0.02)
    x = F.gaussian(rng, cols)
    p = F.quantize_mxfp4(w)
    ref = oracle.matvec(F.MXFP4, p, x, rows, cols, 32)
    out = np.zeros(rows, np.float32)
    hip.KernelTable().matvec_mxfp4(p, x, out, rows, cols, 32)
    assert rel_l2(out, ref) <= REL_L2


_BENCH_EXPERTS = {}


def _experts(rng, n_exp, hidden, eid, bias):
    if (n_exp, hidden, eid, bias) == (32, 2880, 2880, False):
        # config 3: the benchmark's own experts (quantised N(0, 0.02))
        if not _BENCH_EXPERTS:
            _BENCH_EXPERTS["ex"] = F.moe_experts(3, 32, 2880, 2880)
        return _BENCH_EXPERTS["ex"]
    ex = []
    mk = lambda r, c: F.quantize_mxfp4(F.gaussian(rng, (r, c), 0.02))  # noqa: E731
    for _ in range(n_exp):
        e = {"gate": mk(eid, hidden), "up": mk(eid, hidden), "down": mk(hidden, eid)}
        if bias:
            e["gate_bias"] = F.gaussian(rng, eid, 0.1).astype(np.float16).view(np.uint16)
            e["up_bias"] = F.gaussian(rng, eid, 0.1).astype(np.float16).view(np.uint16)
            e["down_bias"] = F.gaussian(rng, hidden, 0.1).astype(np.float16).view(np.uint16)
        ex.append(e)
    return ex


@pytest.mark.parametrize("n_exp,k,hidden,eid,ntok,norm,act,bias", [
    (32, 4, 2880, 2880, 1, 1, 2, False),     # config 3, batch 1
    (32, 4, 2880, 2880, 8, 1, 2, False),     # config 3, batch 8
    (8, 2, 256, 512, 3, 0, 0, True),         # GELU, biases, no renorm
    (4, 4, 128, 64, 8, 1, 3, True),          # every expert picked, ReLU
    (8, 3, 256, 512, 1, 0, 0, True),         # one token (fused down + combine), biases, GELU
    (3, 4, 64, 96, 1, 1, 2, False),          # top-4 of 3 experts: one rank stays empty
    (64, 1, 320, 160, 1, 1, 2, True),        # top-1
    (128, 8, 128, 64, 2, 1, 2, False),       # more experts than lanes: 2 per lane in routing
    (200, 6, 64, 64, 3, 0, 3, True),         # expert count not a multiple of 64, ReLU
])
def test_moe_forward(hip, oracle, n_exp, k, hidden, eid, ntok, norm, act, bias):
    torch = torch_cuda()
    rng = np.random.default_rng(n_exp * 1000 + ntok * 10 + k)
    ex = _experts(rng, n_exp, hidden, eid, bias)
    x = F.gaussian(rng, (ntok, hidden))
    logits = F.gaussian(rng, (ntok, n_exp))
    ref = np.stack([oracle.moe_token(ex, k, norm, act, hidden, eid, x[t], logits[t])
                    for t in range(ntok)])
    tens = {n: [hip.Tensor(e[n], F.MXFP4, *( (eid, hidden) if n != "down" else (hidden, eid)), 32)
                for e in ex] for n in ("gate", "up", "down")}
    biases = {n: ([e[n] for e in ex] if bias else None) for n in ("gate_bias", "up_bias", "down_bias")}
    moe = hip.Moe(tens["gate"], tens["up"], tens["down"], hidden, eid, **biases)
    out = torch.full((ntok, hidden), float("nan"), device="cuda:0")
    moe.forward(k, norm, act, ntok, dev(x), dev(logits), out, stream=_stream())
    got = host(out)
    for t in range(ntok):
        err = rel_l2(got[t], ref[t])
        print(f"moe E={n_exp} k={k} tok {t}: rel_l2={err:.3e}")
        assert err <= REL_L2
    moe.free()
    for ts in tens.values():
        for t in ts:
            t.free()


def test_moe_tie_keeps_lower_expert(hip, oracle):
    """Equal router logits: strict '>' keeps the lower expert ids
    (src/engine.c:994; tests/test_core.c:712-748)."""
    torch = torch_cuda()
    rng = np.random.default_rng(42)
    n_exp, k, hidden, eid = 6, 2, 64, 64
    ex = _experts(rng, n_exp, hidden, eid, False)
    x = F.gaussian(rng, (1, hidden))
    logits = np.zeros((1, n_exp), np.float32)
    ref = oracle.moe_token(ex, k, 1, 2, hidden, eid, x[0], logits[0])
    idx, _ = oracle.topk(oracle.softmax(logits[0]), k, 1)
    assert list(idx) == [0, 1]
    tens = {n: [hip.Tensor(e[n], F.MXFP4, *((eid, hidden) if n != "down" else (hidden, eid)), 32)
                for e in ex] for n in ("gate", "up", "down")}
    moe = hip.Moe(tens["gate"], tens["up"], tens["down"], hidden, eid)
    out = torch.zeros((1, hidden), device="cuda:0")
    moe.forward(k, 1, 2, 1, dev(x), dev(logits), out, stream=_stream())
    assert rel_l2(host(out)[0], ref) <= REL_L2


def test_moe_repeated_calls_reuse_workspace(hip, oracle):
    """One expert table, calls with different token counts and K in a row:
    the workspace (routing list, gate/up and down outputs) is reused and
    every call must still match the oracle.  Calls of more than 8 tokens run
    as consecutive launches of up to 8."""
    torch = torch_cuda()
    rng = np.random.default_rng(7)
    n_exp, hidden, eid = 8, 256, 512
    ex = _experts(rng, n_exp, hidden, eid, True)
    tens = {n: [hip.Tensor(e[n], F.MXFP4, *((eid, hidden) if n != "down" else (hidden, eid)), 32)
                for e in ex] for n in ("gate", "up", "down")}
    biases = {n: [e[n] for e in ex] for n in ("gate_bias", "up_bias", "down_bias")}
    moe = hip.Moe(tens["gate"], tens["up"], tens["down"], hidden, eid, **biases)
    # 20 and 9 tokens: launches of 8, 8, 4 and 8, 1 on one stream and workspace
    for ntok, k in ((8, 4), (1, 2), (5, 3), (8, 8), (2, 1), (20, 4), (9, 2)):
        x = F.gaussian(rng, (ntok, hidden))
        logits = F.gaussian(rng, (ntok, n_exp))
        out = torch.full((ntok, hidden), float("nan"), device="cuda:0")
        moe.forward(k, 1, 2, ntok, dev(x), dev(logits), out, stream=_stream())
        got = host(out)
        for t in range(ntok):
            ref = oracle.moe_token(ex, k, 1, 2, hidden, eid, x[t], logits[t])
            assert rel_l2(got[t], ref) <= REL_L2, (ntok, k, t)
    moe.free()
    for ts in tens.values():
        for t in ts:
            t.free()


@pytest.mark.parametrize("ntok", [1, 8])
def test_moe_stages_one_at_a_time_equal_the_forward(hip, ntok):
    """The measurement switch qsf_hip_moe_stages: forward calls with masks
    1, 2 and 4 in turn (routing, gate/up, down + combine; one token routes
    inside gate/up) leave the same output as one call with 7, bit for bit,
    and a call without the down stage leaves the output untouched."""
    torch = torch_cuda()
    rng = np.random.default_rng(90 + ntok)
    n_exp, k, hidden, eid = 32, 4, 512, 384
    ex = _experts(rng, n_exp, hidden, eid, True)
    tens = {n: [hip.Tensor(e[n], F.MXFP4, *((eid, hidden) if n != "down" else (hidden, eid)), 32)
                for e in ex] for n in ("gate", "up", "down")}
    biases = {n: [e[n] for e in ex] for n in ("gate_bias", "up_bias", "down_bias")}
    moe = hip.Moe(tens["gate"], tens["up"], tens["down"], hidden, eid, **biases)
    x, logits = dev(F.gaussian(rng, (ntok, hidden))), dev(F.gaussian(rng, (ntok, n_exp)))
    full = torch.full((ntok, hidden), float("nan"), device="cuda:0")
    moe.forward(k, 1, 2, ntok, x, logits, full, stream=_stream())
    # other inputs in between, so the workspace holds another call's state
    moe.forward(k, 1, 2, ntok, dev(F.gaussian(rng, (ntok, hidden))), dev(F.gaussian(rng, (ntok, n_exp))),
                torch.empty((ntok, hidden), device="cuda:0"), stream=_stream())
    staged = torch.full((ntok, hidden), float("nan"), device="cuda:0")
    try:
        assert hip.moe_stages(1) == 7
        moe.forward(k, 1, 2, ntok, x, logits, staged, stream=_stream())
        hip.moe_stages(2)
        moe.forward(k, 1, 2, ntok, x, logits, staged, stream=_stream())
        assert np.isnan(host(staged)).all()          # no down stage yet: untouched
        hip.moe_stages(4)
        moe.forward(k, 1, 2, ntok, x, logits, staged, stream=_stream())
    finally:
        assert hip.moe_stages(7) == 4
    assert np.array_equal(host(staged).view(np.uint32), host(full).view(np.uint32))
    moe.free()
    for ts in tens.values():
        for t in ts:
            t.free()


@pytest.mark.parametrize("ntok,all_nan", [(1, False), (3, False), (3, True)])
def test_moe_nan_logits_pick_nothing(hip, oracle, ntok, all_nan):
    """A NaN router logit makes every softmax probability NaN (the sum
    carries it, src/kernels_scalar.c:187-214), and the strict '>' top-K from
    its -1e30 start then picks no expert (src/engine.c:987-1018): that
    token's output is zero.  Token 0 (or every token) has one NaN logit; the
    others are routed as usual.  Covers the no-work paths: the batch-1 fused
    down and the combine."""
    torch = torch_cuda()
    rng = np.random.default_rng(11 + ntok + 5 * all_nan)
    n_exp, k, hidden, eid = 8, 2, 128, 64
    ex = _experts(rng, n_exp, hidden, eid, True)
    x = F.gaussian(rng, (ntok, hidden))
    logits = F.gaussian(rng, (ntok, n_exp))
    for t in range(ntok if all_nan else 1):
        logits[t, 3] = np.nan
    ref = np.stack([oracle.moe_token(ex, k, 1, 2, hidden, eid, x[t], logits[t])
                    for t in range(ntok)])
    assert (ref[0] == 0).all()
    tens = {n: [hip.Tensor(e[n], F.MXFP4, *((eid, hidden) if n != "down" else (hidden, eid)), 32)
                for e in ex] for n in ("gate", "up", "down")}
    biases = {n: [e[n] for e in ex] for n in ("gate_bias", "up_bias", "down_bias")}
    moe = hip.Moe(tens["gate"], tens["up"], tens["down"], hidden, eid, **biases)
    out = torch.full((ntok, hidden), float("nan"), device="cuda:0")
    moe.forward(k, 1, 2, ntok, dev(x), dev(logits), out, stream=_stream())
    got = host(out)
    for t in range(ntok):
        if (ref[t] == 0).all():
            assert (got[t] == 0).all(), t
        else:
            assert rel_l2(got[t], ref[t]) <= REL_L2, t
    moe.free()
    for ts in tens.values():
        for t in ts:
            t.free()
