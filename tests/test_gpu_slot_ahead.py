"""Look-ahead of the table slots (qsf_hip_slot_lookahead).

A slot call that has learnt which weight pointer the engine calls next with
the same x (k after q, up after gate: src/engine.c:848-866, 1118-1125) runs
that successor in its own launch and holds the result for the successor's
call.  What must hold, checked here through the C ABI:
  * every result is bit-identical to the same call made with look-ahead off,
    over several tokens of engine-ordered calls, for chains the kernels can
    group and chains they cannot (their members' launch plans differ);
  * the look-ahead does fire: fewer GEMV launches once learnt;
  * a held result is never served after the successor's weights, the arena
    or x changed between the launching call and the successor's call, or
    when another call came in between.
"""
from __future__ import annotations

import numpy as np
import pytest

from qstream_amd import qsf_format as F
from tests.gpu_util import ENGINES, REL_L2, engine_hip, rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", params=ENGINES, ids=lambda e: f"engine{e}")
def hip(request):
    for h in engine_hip(request):
        old = h.slot_lookahead(-1)
        yield h
        h.slot_lookahead(old)


def _slot(hip, qt):
    kt = hip.KernelTable()
    return {F.Q2: kt.matvec_2bit, F.Q3: kt.matvec_3bit, F.Q4: kt.matvec_4bit,
            F.Q4SYM: kt.matvec_4bit_sym, F.Q2_OUTLIER: kt.matvec_outlier_2bit,
            F.Q4_OUTLIER: kt.matvec_outlier_4bit}[qt]


def _payload(rng, qt, bs, rows, cols):
    w = F.heavy_tail_weights(rng, rows, cols) if qt in (F.Q2_OUTLIER, F.Q4_OUTLIER) else \
        F.gaussian(rng, (rows, cols), 0.02)
    return np.frombuffer(F.quantize_matrix(w, qt, bs), np.uint8).copy()


# (qt, bs, rows) per matrix of a chain sharing x, cols, and whether the
# kernels run the chain as one group (False: the members' plans differ)
CHAINS = {
    "qkv_3bit_bs128": ([(F.Q3, 128, 1024), (F.Q3, 128, 256), (F.Q3, 128, 256)], 2048, True),
    "gate_up_2bit_outlier": ([(F.Q2_OUTLIER, 64, 1100), (F.Q2_OUTLIER, 64, 1107)], 4096, True),
    "qkv_4bit_bs32": ([(F.Q4, 32, 640), (F.Q4, 32, 128), (F.Q4, 32, 128)], 1024, True),
    "gate_up_2bit_bs256": ([(F.Q2, 256, 700), (F.Q2, 256, 700)], 8192, True),
    "gate_up_4sym_bs64": ([(F.Q4SYM, 64, 513), (F.Q4SYM, 64, 513)], 3000, True),
    # a plain 4-bit matrix and an outlier one take different kernels
    "mixed_4bit_outlier": ([(F.Q4, 64, 512), (F.Q4_OUTLIER, 64, 512), (F.Q4, 64, 300)], 4096, False),
}


def _run_tokens(hip, chain, pays, cols, xs):
    outs = []
    for x in xs:
        tok = []
        for (qt, bs, rows), p in zip(chain, pays):
            o = np.full(rows, np.nan, np.float32)
            _slot(hip, qt)(p, x, o, rows, cols, bs)
            tok.append(o)
        outs.append(tok)
    return outs


@pytest.mark.parametrize("name", sorted(CHAINS))
def test_lookahead_bit_identical_and_fires(hip, oracle, name):
    chain, cols, groups = CHAINS[name]
    rng = np.random.default_rng(abs(hash(name)) % 2**32)
    pays = [_payload(rng, qt, bs, rows, cols) for qt, bs, rows in chain]
    xs = [F.gaussian(rng, cols) for _ in range(6)]
    print(f"lookahead case {name}", flush=True)

    hip.slot_lookahead(0)
    alone = _run_tokens(hip, chain, pays, cols, xs)
    for p in pays:
        hip.arena_forget(p)                  # learning starts afresh

    hip.slot_lookahead(2)
    hip.kernel_timing(True)
    ahead = _run_tokens(hip, chain, pays, cols, xs)
    launches = len(hip.kernel_timing_read())
    hip.kernel_timing(False)
    for p in pays:
        hip.arena_forget(p)

    for t, (a, b) in enumerate(zip(alone, ahead)):
        for i, (ya, yb) in enumerate(zip(a, b)):
            assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32)), (name, t, i)
    for i, ((qt, bs, rows), p) in enumerate(zip(chain, pays)):
        ref = oracle.matvec(qt, p.tobytes(), xs[-1], rows, cols, bs)
        assert rel_l2(ahead[-1][i], ref) <= REL_L2
    # learnt after two tokens; then one launch a token when the chain groups
    n = len(chain)
    want = 2 * n + (len(xs) - 2) * (1 if groups else n)
    assert launches == want, (name, launches, want)


def _fresh_single(hip, qt, p, x, rows, cols, bs):
    """The call made alone, on a private copy of the payload."""
    old = hip.slot_lookahead(0)
    q = p.copy()
    o = np.full(rows, np.nan, np.float32)
    _slot(hip, qt)(q, x, o, rows, cols, bs)
    hip.arena_forget(q)
    hip.slot_lookahead(old)
    return o


def test_held_result_never_served_stale(hip, oracle):
    """After the look-ahead has learnt gate -> up, every change between the
    gate call and the up call must reach the up call: its buffer rewritten
    (sampled words change), rewritten under the forget contract, forgotten
    outright, x changed, another call in between (an MXFP4 matvec, a
    different matrix), an unrelated pointer forgotten."""
    qt, bs, rows, cols = F.Q2_OUTLIER, 64, 700, 4096
    rng = np.random.default_rng(77)
    gate = _payload(rng, qt, bs, rows, cols)
    up = _payload(rng, qt, bs, rows + 9, cols)
    other = _payload(rng, qt, bs, 300, cols)
    mx = F.quantize_mxfp4(F.gaussian(rng, (64, cols), 0.02))
    slot = _slot(hip, qt)
    hip.slot_lookahead(2)

    def step(x, between=None):
        og = np.full(rows, np.nan, np.float32)
        slot(gate, x, og, rows, cols, bs)
        if between:
            between(x)
        ou = np.full(rows + 9, np.nan, np.float32)
        slot(up, x, ou, rows + 9, cols, bs)
        return og, ou

    def learn():
        for _ in range(3):
            step(F.gaussian(rng, cols))

    def check_up(x, ou, content):
        want = _fresh_single(hip, qt, content, x, rows + 9, cols, bs)
        assert np.array_equal(ou.view(np.uint32), want.view(np.uint32))
        assert rel_l2(ou, oracle.matvec(qt, content.tobytes(), x, rows + 9, cols, bs)) <= REL_L2

    # 1. up rewritten with new weights (its sampled words change)
    learn()
    new_up = _payload(rng, qt, bs, rows + 9, cols)
    assert new_up.size == up.size
    x = F.gaussian(rng, cols)
    keep = up.copy()
    _, ou = step(x, lambda _x: up.__setitem__(slice(None), new_up))
    check_up(x, ou, new_up)
    assert not np.array_equal(ou, _fresh_single(hip, qt, keep, x, rows + 9, cols, bs))
    # (up is volatile now: forget it so that it is learnt again)
    hip.arena_forget(up)

    # 2. one unsampled byte rewritten under the contract (forget first)
    learn()
    x = F.gaussian(rng, cols)
    edited = up.copy()
    edited[edited.size // 16] ^= 0x5A

    def rewrite_and_forget(_x):
        up[:] = edited
        assert hip.arena_forget(up)
    _, ou = step(x, rewrite_and_forget)
    check_up(x, ou, edited)

    # 3. up forgotten outright (no change of content)
    learn()
    x = F.gaussian(rng, cols)
    _, ou = step(x, lambda _x: hip.arena_forget(up))
    check_up(x, ou, up)

    # 4. x changed between the two calls
    learn()
    x = F.gaussian(rng, cols)
    x2 = x.copy()
    x2[17] += 0.25
    og = np.full(rows, np.nan, np.float32)
    slot(gate, x, og, rows, cols, bs)
    ou = np.full(rows + 9, np.nan, np.float32)
    slot(up, x2, ou, rows + 9, cols, bs)
    check_up(x2, ou, up)

    # 5. an MXFP4 call on the same x in between
    learn()
    x = F.gaussian(rng, cols)
    om = np.full(64, np.nan, np.float32)
    _, ou = step(x, lambda xx: hip.KernelTable().matvec_mxfp4(mx, xx, om, 64, cols, 32))
    check_up(x, ou, up)
    assert rel_l2(om, oracle.matvec(F.MXFP4, mx, x, 64, cols, 32)) <= REL_L2

    # 6. another matrix on the same x in between (gate's successor changes)
    learn()
    x = F.gaussian(rng, cols)
    oo = np.full(300, np.nan, np.float32)
    _, ou = step(x, lambda xx: slot(other, xx, oo, 300, cols, bs))
    check_up(x, ou, up)
    assert rel_l2(oo, oracle.matvec(qt, other.tobytes(), x, 300, cols, bs)) <= REL_L2

    # 7. an unrelated pointer forgotten in between
    learn()
    x = F.gaussian(rng, cols)
    _, ou = step(x, lambda _x: hip.arena_forget(other))
    check_up(x, ou, up)

    for p in (gate, up, other):
        hip.arena_forget(p)


def test_lookahead_setting(hip):
    old = hip.slot_lookahead(3)
    assert hip.slot_lookahead(-1) == 3
    assert hip.slot_lookahead(100) == 3
    assert hip.slot_lookahead(-1) == 7
    hip.slot_lookahead(old)
