"""GPU parity of the device-resident decode glue (decode_glue.hip) and of
the logits / embedding path, against the oracle's restatements of
src/engine.c and src/kernels_scalar.c, through the C ABI.

Bit-exact: the int8 KV codes and scales, attention at a single position
(softmax weight exactly 1), the residual add and its NaN index, the
embedding rows.  Otherwise rel-L2 <= 1e-5 (fp32 sums in a different order,
device exp/cos/sin/tanh within an ulp or two of the C library's).
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


def _s():
    return torch_cuda().cuda.current_stream()


@pytest.mark.parametrize("dim", [7, 4096, 5120, 11008])
def test_norms(hip, oracle, dim):
    torch = torch_cuda()
    rng = np.random.default_rng(dim)
    x = (rng.standard_normal(dim) * 3).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    b = (0.1 * rng.standard_normal(dim)).astype(np.float32)
    out = torch.empty(dim, device="cuda:0")
    hip.rms_norm(dev(x), out, dev(w), 1e-5, stream=_s())
    assert rel_l2(host(out), oracle.rms_norm(x, w, 1e-5)) <= REL_L2
    for bias in (None, b):
        hip.layer_norm(dev(x), out, dev(w), None if bias is None else dev(bias), 1e-6, stream=_s())
        assert rel_l2(host(out), oracle.layer_norm(x, w, bias, 1e-6)) <= REL_L2


@pytest.mark.parametrize("position", [0, 1, 4095, 100000])
def test_rope(hip, oracle, position):
    rng = np.random.default_rng(position + 1)
    hd, nh, nkv, theta = 128, 32, 8, 500000.0
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal(nkv * hd).astype(np.float32)
    rq, rk = oracle.rope(q, k, hd, position, theta, nh, nkv)
    r = hip.Rope(hd, theta)
    dq, dk = dev(q), dev(k)
    r.apply(dq, dk, nh, nkv, position, stream=_s())
    gq, gk = host(dq), host(dk)
    r.free()
    print(f"rope position {position}: q {rel_l2(gq, rq):.2e} k {rel_l2(gk, rk):.2e}")
    assert rel_l2(gq, rq) <= REL_L2 and rel_l2(gk, rk) <= REL_L2
    if position == 0:
        assert np.array_equal(gq, q) and np.array_equal(gk, k)


def test_kv_store_bit_exact(hip, oracle):
    torch = torch_cuda()
    rng = np.random.default_rng(2)
    nkv, hd, max_seq = 8, 128, 64
    kc = np.zeros((nkv, max_seq, hd), np.int8)
    vc = np.zeros_like(kc)
    ks = np.zeros((nkv, max_seq), np.float32)
    vs = np.zeros_like(ks)
    dkc, dvc = dev(kc), dev(vc)
    dks, dvs = dev(ks), dev(vs)
    for pos in (0, 5, 63):
        k = (rng.standard_normal(nkv * hd) * (pos + 1)).astype(np.float32)
        v = (rng.standard_normal(nkv * hd) * 0.01).astype(np.float32)
        k[hd * 3:hd * 4] = 0.0                       # an all-zero head
        k[hd * 5:hd * 6] = 1e-31                     # absmax below the 1e-30 floor: zeros
        oracle.kv_store(kc, vc, ks, vs, max_seq, nkv, hd, pos, k, v)
        hip.kv_store(dkc, dvc, dks, dvs, max_seq, nkv, hd, pos, dev(k), dev(v), stream=_s())
    torch.cuda.synchronize()
    assert np.array_equal(host(dkc), kc) and np.array_equal(host(dvc), vc)
    assert np.array_equal(host(dks).view(np.uint32), ks.view(np.uint32))
    assert np.array_equal(host(dvs).view(np.uint32), vs.view(np.uint32))


def test_kv_store_exact_ties(hip):
    """Exact .5 ties and the 0.5 - 2^-25 case of the reference's
    truncating rounding (src/engine.c:265,287), known answers pinned in
    tests/test_oracle_glue.py, in every head of a 128-wide store."""
    from tests.test_oracle_glue import KV_TIE_CODES, KV_TIE_ROW
    torch = torch_cuda()
    nkv, hd, max_seq, pos = 4, 128, 8, 3
    k = np.tile(KV_TIE_ROW, nkv * hd // 16).astype(np.float32)
    dkc = dev(np.zeros((nkv, max_seq, hd), np.int8))
    dvc = dev(np.zeros((nkv, max_seq, hd), np.int8))
    dks, dvs = dev(np.zeros((nkv, max_seq), np.float32)), dev(np.zeros((nkv, max_seq), np.float32))
    hip.kv_store(dkc, dvc, dks, dvs, max_seq, nkv, hd, pos, dev(k), dev(-k), stream=_s())
    torch.cuda.synchronize()
    want = np.tile(KV_TIE_CODES, hd // 16)
    for h in range(nkv):
        assert np.array_equal(host(dkc)[h, pos], want) and np.array_equal(host(dvc)[h, pos], -want)
    assert np.all(host(dks)[:, pos] == 1.0) and np.all(host(dvs)[:, pos] == 1.0)


# head_dim 64, 128 and 256 take the load-everything-first kernel, others the
# general one; positions 129 and 300 leave a partial last chunk of 128
@pytest.mark.parametrize("nh,nkv,hd,position", [(32, 32, 128, 0), (32, 32, 128, 1023),
                                                (32, 8, 128, 300), (8, 2, 64, 4095),
                                                (32, 8, 128, 129), (4, 4, 256, 700),
                                                (6, 2, 80, 200), (2, 1, 64, 0)])
def test_attention(hip, oracle, nh, nkv, hd, position):
    torch = torch_cuda()
    rng = np.random.default_rng(nh + position)
    max_seq = position + 3
    kc = rng.integers(-127, 128, (nkv, max_seq, hd)).astype(np.int8)
    vc = rng.integers(-127, 128, (nkv, max_seq, hd)).astype(np.int8)
    ks = (rng.random((nkv, max_seq)) * 0.05).astype(np.float32)
    vs = (rng.random((nkv, max_seq)) * 0.05).astype(np.float32)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    ref = oracle.attention(q, kc, vc, ks, vs, max_seq, nh, nkv, hd, position)
    out = torch.full((nh * hd,), float("nan"), device="cuda:0")
    hip.attention(dev(q), dev(kc), dev(vc), dev(ks), dev(vs), max_seq, nh, nkv, hd, position, out,
                  stream=_s())
    got = host(out)
    err = rel_l2(got, ref)
    print(f"attention nh {nh} nkv {nkv} hd {hd} pos {position}: rel_l2 {err:.2e}")
    assert err <= REL_L2
    if position == 0:        # softmax of one score is exactly 1
        assert np.array_equal(got, ref)


@pytest.mark.parametrize("act", [2, 0, 3])
def test_act_mul(hip, oracle, act):
    rng = np.random.default_rng(act)
    n = 11008
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    ref = oracle.vec_mul(oracle.act(act, g), u)
    dg = dev(g)
    hip.act_mul(dg, dev(u), act, stream=_s())
    got = host(dg)
    assert rel_l2(got, ref) <= REL_L2
    if act == 3:
        assert np.array_equal(got, ref)


def test_residual_and_nan_check(hip, oracle):
    torch = torch_cuda()
    rng = np.random.default_rng(4)
    n = 4096
    res = rng.standard_normal(n).astype(np.float32)
    bad = torch.full((1,), 12345, dtype=torch.int32, device="cuda:0")
    for case in range(4):
        x = rng.standard_normal(n).astype(np.float32)
        if case == 1:
            x[2000] = np.nan
            x[3000] = np.inf
        if case == 2:
            x[17] = 2e30
        if case == 3:
            x[:] = 0
            x[5] = np.float32(1e30) - res[5]            # lands near, not beyond, 1e30
        want, want_bad = oracle.residual_check(res, x)
        d = dev(res)
        hip.residual(d, dev(x), bad, stream=_s())
        assert np.array_equal(host(d).view(np.uint32), want.view(np.uint32))
        assert int(host(bad)[0]) == want_bad, case
        d2 = dev(res)
        hip.residual(d2, dev(x), None, stream=_s())        # no check: add only
        assert np.array_equal(host(d2).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("qt,bs,hd", [(F.Q4, 64, 4096), (F.Q2, 32, 100), (F.Q3, 128, 300),
                                      (F.Q4SYM, 64, 96)])
def test_embed_row_bit_exact(hip, oracle, qt, bs, hd):
    torch = torch_cuda()
    rng = np.random.default_rng(qt + hd)
    vocab = 50
    table = F.quantize_matrix(F.gaussian(rng, (vocab, hd), 0.02), qt, bs)
    t = hip.Tensor(table, qt, vocab, hd, bs)
    out = torch.empty(hd, device="cuda:0")
    for token in (0, 17, vocab - 1):
        hip.embed_row(t, token, out, stream=_s())
        want = oracle.embed_row(qt, table, bs, hd, token)
        assert np.array_equal(host(out).view(np.uint32), want.view(np.uint32))
    t.free()
    with pytest.raises(hip.QsfHipError):
        t2 = hip.Tensor(table, qt, vocab, hd, bs)
        try:
            hip.embed_row(t2, vocab, out)                   # token out of range
        finally:
            t2.free()


def test_embed_row_fp16(hip, oracle):
    torch = torch_cuda()
    rng = np.random.default_rng(7)
    vocab, hd = 40, 70
    table = F.gaussian(rng, (vocab, hd), 0.5).astype(np.float16)
    out = torch.empty(hd, device="cuda:0")
    dt = dev(table.view(np.uint16).reshape(-1))
    for token in (0, 39):
        hip.embed_row_fp16(dt, hd, token, out, stream=_s())
        want = oracle.embed_row(7, table.view(np.uint8).reshape(-1), 64, hd, token)
        assert np.array_equal(host(out).view(np.uint32), want.view(np.uint32))


# ---- logits at vocabulary shape (src/engine.c:1199-1244) --------------------
@pytest.mark.parametrize("vocab,qt", [(32000, F.Q4), (128256, F.Q4), (32000, F.Q2)])
def test_logits_matvec_vocab_shape(hip, oracle, vocab, qt):
    """The tied-embedding / output-head matvec: vocab x 4096 through the same
    slot the engine calls (get_matvec_fn on the table's type)."""
    rng = np.random.default_rng(vocab + qt)
    hd, bs = 4096, 64
    table = F.quantize_matrix(F.gaussian(rng, (vocab, hd), 0.02), qt, bs)
    x = F.gaussian(rng, hd)
    ref = oracle.matvec(qt, table, x, vocab, hd, bs)
    t = hip.Tensor(table, qt, vocab, hd, bs)
    y = torch_cuda().full((vocab,), float("nan"), device="cuda:0")
    t.matvec(dev(x), y, stream=_s())
    err = rel_l2(host(y), ref)
    t.free()
    print(f"logits {vocab}x{hd} type {qt}: rel_l2 {err:.2e}")
    assert err <= REL_L2


# ---- one decoder layer, device-resident, over several positions --------------
def test_device_resident_layer_chain(hip, oracle):
    """A small LLaMA-style layer (RMSNorm, q/k/v, RoPE, int8 KV cache,
    attention, o, residual, RMSNorm, gate/up, SiLU x up, down, residual +
    NaN check) run entirely on the device for five consecutive positions,
    against the same chain through the oracle.  The int8 re-quantisation of
    k and v can move a code by one step when the two sides' k differ in the
    last fp32 bit, so the chain is held to 1e-4 (each kernel alone is held
    to 1e-5 or bit-exact above)."""
    torch = torch_cuda()
    rng = np.random.default_rng(11)
    hid, nh, nkv, hd, eid, bs, qt, max_seq, eps = 256, 4, 2, 64, 512, 64, F.Q4, 16, 1e-5
    shapes = {"q": (nh * hd, hid), "k": (nkv * hd, hid), "v": (nkv * hd, hid), "o": (hid, nh * hd),
              "gate": (eid, hid), "up": (eid, hid), "down": (hid, eid)}
    pay = {n: F.quantize_matrix(F.gaussian(rng, s, 0.05), qt, bs) for n, s in shapes.items()}
    T = {n: hip.Tensor(pay[n], qt, *shapes[n], bs) for n in shapes}
    an_w = (1 + 0.1 * rng.standard_normal(hid)).astype(np.float32)
    fn_w = (1 + 0.1 * rng.standard_normal(hid)).astype(np.float32)
    rope = hip.Rope(hd, 10000.0)
    # oracle state
    okc = np.zeros((nkv, max_seq, hd), np.int8)
    ovc = np.zeros_like(okc)
    oks = np.zeros((nkv, max_seq), np.float32)
    ovs = np.zeros_like(oks)
    # device state
    dkc, dvc, dks, dvs = dev(okc), dev(ovc), dev(oks), dev(ovs)
    d = {n: torch.empty(shapes[n][0], device="cuda:0") for n in shapes}
    dx, dattn = torch.empty(hid, device="cuda:0"), torch.empty(nh * hd, device="cuda:0")
    bad = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    s = _s()
    for pos in range(5):
        emb = rng.standard_normal(hid).astype(np.float32)
        # oracle chain (src/engine.c:805-1187)
        res = emb.copy()
        x = oracle.rms_norm(res, an_w, eps)
        q, k, v = (oracle.matvec(qt, pay[n], x, *shapes[n], bs) for n in ("q", "k", "v"))
        q, k = oracle.rope(q, k, hd, pos, 10000.0, nh, nkv)
        oracle.kv_store(okc, ovc, oks, ovs, max_seq, nkv, hd, pos, k, v)
        attn = oracle.attention(q, okc, ovc, oks, ovs, max_seq, nh, nkv, hd, pos)
        res, _ = oracle.residual_check(res, oracle.matvec(qt, pay["o"], attn, *shapes["o"], bs))
        x = oracle.rms_norm(res, fn_w, eps)
        g = oracle.matvec(qt, pay["gate"], x, *shapes["gate"], bs)
        u = oracle.matvec(qt, pay["up"], x, *shapes["up"], bs)
        h = oracle.vec_mul(oracle.act(2, g), u)
        res, want_bad = oracle.residual_check(res, oracle.matvec(qt, pay["down"], h, *shapes["down"], bs))
        # device chain: no host round trip between the launches
        dres = dev(emb)
        hip.rms_norm(dres, dx, dev(an_w), eps, stream=s)
        hip.matvec_group([T["q"]], dx, [d["q"]], stream=s)
        hip.matvec_group([T["k"], T["v"]], dx, [d["k"], d["v"]], stream=s)
        rope.apply(d["q"], d["k"], nh, nkv, pos, stream=s)
        hip.kv_store(dkc, dvc, dks, dvs, max_seq, nkv, hd, pos, d["k"], d["v"], stream=s)
        hip.attention(d["q"], dkc, dvc, dks, dvs, max_seq, nh, nkv, hd, pos, dattn, stream=s)
        hip.matvec_group([T["o"]], dattn, [d["o"]], stream=s)
        hip.residual(dres, d["o"], None, stream=s)
        hip.rms_norm(dres, dx, dev(fn_w), eps, stream=s)
        hip.matvec_group([T["gate"], T["up"]], dx, [d["gate"], d["up"]], stream=s)
        hip.act_mul(d["gate"], d["up"], 2, stream=s)
        hip.matvec_group([T["down"]], d["gate"], [d["down"]], stream=s)
        hip.residual(dres, d["down"], bad, stream=s)
        err = rel_l2(host(dres), res)
        print(f"layer chain position {pos}: rel_l2 {err:.2e}")
        assert err <= 1e-4
        assert int(host(bad)[0]) == want_bad == -1
    rope.free()
    for t in T.values():
        t.free()


# ---- fused launches: bit-identical to the separate calls ------------------------
@pytest.mark.parametrize("layer_norm,with_bias", [(False, False), (True, False), (True, True)])
@pytest.mark.parametrize("poison", [None, "nan", "big"])
def test_residual_norm_equals_separate_calls(hip, layer_norm, with_bias, poison):
    torch = torch_cuda()
    rng = np.random.default_rng(7 + 2 * layer_norm + with_bias)
    n = 4096
    res = rng.standard_normal(n).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    if poison == "nan":
        x[1234] = np.nan
    elif poison == "big":
        x[77] = 3e30
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    b = (0.1 * rng.standard_normal(n)).astype(np.float32) if with_bias else None
    eps = 1e-5
    r1, r2 = dev(res), dev(res)
    o1, o2 = torch.empty(n, device="cuda:0"), torch.empty(n, device="cuda:0")
    bad1 = torch.full((1,), 7, dtype=torch.int32, device="cuda:0")
    bad2 = bad1.clone()
    hip.residual(r1, dev(x), bad1, stream=_s())
    if layer_norm:
        hip.layer_norm(r1, o1, dev(w), None if b is None else dev(b), eps, stream=_s())
    else:
        hip.rms_norm(r1, o1, dev(w), eps, stream=_s())
    hip.residual_norm(r2, dev(x), dev(w), eps, o2, bad=bad2, b=None if b is None else dev(b),
                      layer_norm=layer_norm, stream=_s())
    assert np.array_equal(host(r1).view(np.uint32), host(r2).view(np.uint32))
    assert np.array_equal(host(o1).view(np.uint32), host(o2).view(np.uint32))
    assert int(host(bad1)[0]) == int(host(bad2)[0]) == {None: -1, "nan": 1234, "big": 77}[poison]


@pytest.mark.parametrize("nh,nkv,hd,position", [(32, 32, 128, 1023), (32, 8, 128, 5), (8, 2, 64, 300),
                                                (4, 4, 256, 77), (6, 2, 80, 0)])
def test_rope_kv_store_equals_separate_calls(hip, nh, nkv, hd, position):
    torch = torch_cuda()
    rng = np.random.default_rng(nh + hd + position)
    max_seq = position + 4
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal(nkv * hd).astype(np.float32)
    v = rng.standard_normal(nkv * hd).astype(np.float32)
    k[:hd] = 0.0                               # a zero head: scale 0, codes 0
    rope = hip.Rope(hd, 10000.0)
    outs = []
    for fused in (False, True):
        dq, dk, dv = dev(q), dev(k), dev(v)
        kc = torch.full((nkv, max_seq, hd), 5, dtype=torch.int8, device="cuda:0")
        vc = kc.clone()
        ks = torch.full((nkv, max_seq), 0.5, device="cuda:0")
        vs = ks.clone()
        if fused:
            rope.apply_and_store(dq, dk, dv, nh, nkv, position, kc, vc, ks, vs, max_seq, stream=_s())
        else:
            rope.apply(dq, dk, nh, nkv, position, stream=_s())
            hip.kv_store(kc, vc, ks, vs, max_seq, nkv, hd, position, dk, dv, stream=_s())
        outs.append([host(a).view(np.uint8) for a in (dq, dk, kc, vc, ks, vs)])
    for name, a, c in zip(("q", "k", "kc", "vc", "ks", "vs"), *outs):
        assert np.array_equal(a, c), name


@pytest.mark.parametrize("nh,nkv,hd,position", [(32, 32, 128, 1023), (32, 8, 128, 127), (32, 8, 128, 128),
                                                (8, 2, 64, 300), (8, 8, 64, 0), (4, 4, 256, 77),
                                                (4, 2, 256, 256), (16, 4, 256, 2050), (6, 2, 80, 130)])
def test_rope_kv_attention_equals_separate_calls(hip, nh, nkv, hd, position):
    """RoPE + KV store + attention in one call (two launches for head_dim
    64/128/256, the new row's codes used from LDS) against the RoPE + KV
    store launch followed by attention: the cache row, the scales and the
    attention output bit for bit, the older rows untouched.  Positions at a
    chunk's first row (128, 256, 0) and last (127), GQA and MHA; hd 80 runs
    the two-call path."""
    torch = torch_cuda()
    rng = np.random.default_rng(3 * nh + hd + position)
    max_seq = position + 3
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal(nkv * hd).astype(np.float32)
    v = rng.standard_normal(nkv * hd).astype(np.float32)
    k[:hd] = 0.0                               # a zero head: scale 0, codes 0
    v[-hd:] *= 1e3                             # a large one
    kc0 = rng.integers(-127, 128, (nkv, max_seq, hd), dtype=np.int8)
    vc0 = rng.integers(-127, 128, (nkv, max_seq, hd), dtype=np.int8)
    ks0 = (0.02 * rng.random((nkv, max_seq))).astype(np.float32)
    vs0 = (0.02 * rng.random((nkv, max_seq))).astype(np.float32)
    rope = hip.Rope(hd, 500000.0)
    outs = []
    for fused in (False, True):
        dq, dk, dv = dev(q), dev(k), dev(v)
        kc, vc, ks, vs = (torch.from_numpy(a.copy()).to("cuda:0") for a in (kc0, vc0, ks0, vs0))
        out = torch.full((nh * hd,), np.nan, device="cuda:0")
        if fused:
            rope.apply_store_attend(dq, dk, dv, nh, nkv, position, kc, vc, ks, vs, max_seq, out, stream=_s())
        else:
            rope.apply_and_store(dq, dk, dv, nh, nkv, position, kc, vc, ks, vs, max_seq, stream=_s())
            hip.attention(dq, kc, vc, ks, vs, max_seq, nh, nkv, hd, position, out, stream=_s())
        outs.append([host(a).view(np.uint8) for a in (kc, vc, ks, vs, out)])
    for name, a, c in zip(("kc", "vc", "ks", "vs", "out"), *outs):
        assert np.array_equal(a, c), name
    kc1 = outs[1][0].view(np.int8).reshape(nkv, max_seq, hd)
    keep = np.ones(max_seq, bool)
    keep[position] = False
    assert np.array_equal(kc1[:, keep], kc0[:, keep])
    assert not kc1[0, position].any()          # the zero head
    assert np.isfinite(outs[1][4].view(np.float32)).all()
    rope.free()
