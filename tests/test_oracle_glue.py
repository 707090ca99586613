"""Pinning the oracle's decode-glue restatements (CPU only).

* Functions that live in src/kernels_scalar.c (norms, softmax, activations,
  vector add/mul) are compared bit for bit with the reference's own
  translation unit compiled strictly into oracle/_ref.
* The static helpers apply_rope and kv_cache_store of src/engine.c are
  compared bit for bit with the reference's engine.c compiled strictly into
  oracle/_ref (oracle/ref_glue.c includes the unit and exports them).
* The rest of the engine's inline glue (the attention loop, the residual
  NaN check, the embedding lookup) lives inside qsf_forward and cannot be
  called alone, so it is pinned by closed forms, invariants and fp64 brute
  force, chosen so that a wrong sign, pairing, index or rounding rule
  fails; so are RoPE and the KV store as well.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from qstream_amd import qsf_format as F


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


# ---- against the compiled reference (bit-exact) -----------------------------
@pytest.mark.parametrize("dim", [1, 7, 4096, 5120])
def test_norms_bit_exact_vs_reference(oracle, ref, dim):
    rng = np.random.default_rng(dim)
    x = (rng.standard_normal(dim) * 3).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    b = (0.1 * rng.standard_normal(dim)).astype(np.float32)
    for eps in (1e-5, 1e-6):
        want = np.empty(dim, np.float32)
        ref.lib.qsf_rms_norm_scalar(_p(x), _p(want), _p(w), None, dim, eps)
        assert np.array_equal(oracle.rms_norm(x, w, eps).view(np.uint32), want.view(np.uint32))
        for bias in (None, b):
            ref.lib.qsf_layer_norm_scalar(_p(x), _p(want), _p(w), None if bias is None else _p(bias),
                                          dim, eps)
            got = oracle.layer_norm(x, w, bias, eps)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_softmax_activations_vecops_bit_exact_vs_reference(oracle, ref):
    rng = np.random.default_rng(5)
    for n in (1, 3, 64, 1000, 4097):
        x = (rng.standard_normal(n) * 8).astype(np.float32)
        want = np.empty(n, np.float32)
        ref.lib.qsf_softmax_scalar(_p(x), _p(want), n)
        assert np.array_equal(oracle.softmax(x).view(np.uint32), want.view(np.uint32))
        for act, name in ((2, "qsf_silu_scalar"), (0, "qsf_gelu_scalar"), (3, "qsf_relu_scalar")):
            want = x.copy()
            getattr(ref.lib, name)(_p(want), n)
            assert np.array_equal(oracle.act(act, x).view(np.uint32), want.view(np.uint32)), name
        y = rng.standard_normal(n).astype(np.float32)
        for fn, name in ((oracle.vec_add, "qsf_vec_add_scalar_impl"),
                         (oracle.vec_mul, "qsf_vec_mul_scalar_impl")):
            want = np.empty(n, np.float32)
            getattr(ref.lib, name)(_p(x), _p(y), _p(want), n)
            assert np.array_equal(fn(x, y).view(np.uint32), want.view(np.uint32)), name


# ---- RoPE: closed form --------------------------------------------------------
@pytest.fixture(scope="module")
def ref_glue():
    from oracle.oracle import ref_glue as rg
    r = rg()
    if r is None:
        pytest.skip("oracle/_ref not built (reference sources absent)")
    return r


@pytest.mark.parametrize("hd,nh,nkv,position,theta", [(128, 32, 8, 0, 10000.0), (128, 4, 4, 1023, 10000.0),
                                                      (64, 8, 2, 77777, 500000.0), (256, 2, 1, 5, 1e6),
                                                      (80, 6, 2, 131071, 10000.0), (2, 3, 1, 9, 10000.0)])
def test_rope_bit_exact_vs_reference(oracle, ref_glue, hd, nh, nkv, position, theta):
    """apply_rope of the reference's engine.c against the oracle's restatement:
    every bit of q and k, large positions included (the angle reduction)."""
    rng = np.random.default_rng(hd + position)
    q = (rng.standard_normal(nh * hd) * 3).astype(np.float32)
    k = (rng.standard_normal(nkv * hd) * 3).astype(np.float32)
    q1, k1 = oracle.rope(q, k, hd, position, theta, nh, nkv)
    q2, k2 = ref_glue.rope(q, k, hd, position, theta, nh, nkv)
    assert np.array_equal(q1.view(np.uint32), q2.view(np.uint32))
    assert np.array_equal(k1.view(np.uint32), k2.view(np.uint32))


@pytest.mark.parametrize("nkv,hd,max_seq,position,scale", [(8, 128, 16, 5, 1.0), (2, 64, 4, 3, 1e-3),
                                                           (3, 256, 2, 0, 50.0), (1, 80, 9, 8, 1.0)])
def test_kv_store_bit_exact_vs_reference(oracle, ref_glue, nkv, hd, max_seq, position, scale):
    """kv_cache_store of the reference's engine.c against the oracle's: codes
    and scales bit for bit, with a zero head, a tiny head (absmax below
    1e-30), exact .5 ties and values that round up to a tie, and the rows
    around the stored one left alone."""
    rng = np.random.default_rng(nkv * hd + position)
    k = (rng.standard_normal(nkv * hd) * scale).astype(np.float32)
    v = (rng.standard_normal(nkv * hd) * scale).astype(np.float32)
    k[:hd] = 0.0                                  # a zero head
    if nkv > 1:
        v[hd:2 * hd] = 1e-31                      # absmax below 1e-30: codes 0
    n = min(hd, len(KV_TIE_ROW))
    v[-hd:-hd + n] = KV_TIE_ROW[:n]               # ties and near-ties (absmax 127: inv 1)
    outs = []
    for impl in (oracle, ref_glue):
        kc = np.full((nkv, max_seq, hd), 7, np.int8)
        vc = kc.copy()
        ks = np.full((nkv, max_seq), 0.25, np.float32)
        vs = ks.copy()
        impl.kv_store(kc, vc, ks, vs, max_seq, nkv, hd, position, k, v)
        outs.append((kc, vc, ks.view(np.uint32), vs.view(np.uint32)))
    for a, b in zip(*outs):
        assert np.array_equal(a, b)


def rope_freqs(head_dim, theta):
    """The reference's fp32 frequencies 1.0f / powf(theta, (float)i / head_dim)
    with the C library's powf (src/engine.c:210)."""
    libm = C.CDLL("libm.so.6")
    libm.powf.restype = C.c_float
    libm.powf.argtypes = [C.c_float, C.c_float]
    return np.array([np.float32(1.0) / np.float32(libm.powf(theta, np.float32(i) / np.float32(head_dim)))
                     for i in range(0, head_dim, 2)], np.float32)


def _rope_f64(h, head_dim, position, theta):
    """Pair (2j, 2j+1) rotated by position * freq_j with the reference's fp32
    frequency; angle reduction and rotation in fp64."""
    h = h.astype(np.float64).reshape(-1, head_dim)
    freq = rope_freqs(head_dim, theta).astype(np.float64)
    ang = np.fmod(position * freq, 2 * np.pi)
    c, s = np.cos(ang), np.sin(ang)
    out = h.copy()
    out[:, 0::2] = h[:, 0::2] * c - h[:, 1::2] * s
    out[:, 1::2] = h[:, 0::2] * s + h[:, 1::2] * c
    return out.reshape(-1)


@pytest.mark.parametrize("position", [0, 1, 17, 4095, 100000])
def test_rope_closed_form(oracle, position):
    rng = np.random.default_rng(position)
    hd, nh, nkv, theta = 128, 4, 2, 10000.0
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal(nkv * hd).astype(np.float32)
    q2, k2 = oracle.rope(q, k, hd, position, theta, nh, nkv)
    if position == 0:
        assert np.array_equal(q2, q) and np.array_equal(k2, k)
    for a, b in ((q, q2), (k, k2)):
        want = _rope_f64(a, hd, position, theta)
        assert np.max(np.abs(b - want)) <= 2e-6 * (1 + np.abs(want).max())
        # each pair keeps its length
        n0 = np.hypot(a[0::2].astype(np.float64), a[1::2])
        n1 = np.hypot(b[0::2].astype(np.float64), b[1::2])
        assert np.allclose(n0, n1, rtol=1e-6, atol=1e-7)


# ---- int8 KV store: invariants and brute force -------------------------------
def test_kv_store_invariants(oracle):
    rng = np.random.default_rng(9)
    nkv, hd, max_seq, pos = 3, 64, 16, 5
    kc = np.zeros((nkv, max_seq, hd), np.int8)
    vc = np.zeros_like(kc)
    ks = np.zeros((nkv, max_seq), np.float32)
    vs = np.zeros_like(ks)
    k = (rng.standard_normal(nkv * hd) * 2).astype(np.float32)
    v = (rng.standard_normal(nkv * hd) * 0.1).astype(np.float32)
    v[hd:2 * hd] = 0.0                       # an all-zero head: scale 0, codes 0
    oracle.kv_store(kc, vc, ks, vs, max_seq, nkv, hd, pos, k, v)
    others = np.ones(max_seq, bool)
    others[pos] = False
    assert not kc[:, others].any() and not vc[:, others].any()      # only row `pos` written
    for src, cache, sc in ((k, kc, ks), (v, vc, vs)):
        for h in range(nkv):
            row = src[h * hd:(h + 1) * hd]
            amax = np.float32(np.abs(row).max())
            assert sc[h, pos] == np.float32(amax / np.float32(127.0))
            codes = cache[h, pos].astype(np.int32)
            if amax == 0:
                assert not codes.any()
                continue
            assert np.abs(codes).max() == 127 and codes[np.argmax(np.abs(row))] == np.sign(
                row[np.argmax(np.abs(row))]) * 127
            # nearest code, ties away from zero: |x*127/amax - code| <= 1/2
            t = row.astype(np.float64) * 127.0 / float(amax)
            assert np.all(np.abs(t - codes) <= 0.5 + 1e-5)
            assert np.all(np.sign(codes[codes != 0]) == np.sign(row[codes != 0]))


# Exact ties of the int8 KV code.  With |max| = 127 the scale 127/amax is
# exactly 1, so each value reaches the rounding as written.  The reference
# rounds by truncating v +- 0.5f in fp32 (src/engine.c:265,287): halves go
# away from zero (2.5 -> 3, where half-to-even gives 2), and 0.5 - 2^-25
# goes to 1, because v + 0.5f rounds up to 1.0f before the truncation.
KV_TIE_ROW = np.array([127.0, 2.5, -2.5, 0.5, -0.5, 3.5, -3.5, 126.5, -126.5, 0.25, -0.25,
                       0.5 - 2.0 ** -25, -(0.5 - 2.0 ** -25), 2.5 - 2.0 ** -22, 1.5, -1.5], np.float32)
KV_TIE_CODES = np.array([127, 3, -3, 1, -1, 4, -4, 127, -127, 0, 0, 1, -1, 2, 2, -2], np.int8)


def test_kv_store_exact_ties(oracle):
    hd = 16
    kc = np.zeros((1, 2, hd), np.int8)
    vc = np.zeros_like(kc)
    ks = np.zeros((1, 2), np.float32)
    vs = np.zeros_like(ks)
    oracle.kv_store(kc, vc, ks, vs, 2, 1, hd, 1, KV_TIE_ROW, -KV_TIE_ROW)
    assert np.array_equal(kc[0, 1], KV_TIE_CODES) and np.array_equal(vc[0, 1], -KV_TIE_CODES)
    assert ks[0, 1] == vs[0, 1] == np.float32(1.0)


# ---- attention: fp64 brute force ---------------------------------------------
@pytest.mark.parametrize("nh,nkv,position", [(4, 4, 0), (4, 4, 9), (8, 2, 30)])
def test_attention_vs_fp64(oracle, nh, nkv, position):
    rng = np.random.default_rng(nh * 100 + position)
    hd, max_seq = 32, 40
    kc = rng.integers(-127, 128, (nkv, max_seq, hd)).astype(np.int8)
    vc = rng.integers(-127, 128, (nkv, max_seq, hd)).astype(np.int8)
    ks = (rng.random((nkv, max_seq)) * 0.02).astype(np.float32)
    vs = (rng.random((nkv, max_seq)) * 0.02).astype(np.float32)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    got = oracle.attention(q, kc, vc, ks, vs, max_seq, nh, nkv, hd, position)
    want = np.zeros((nh, hd))
    for h in range(nh):
        g = h // (nh // nkv)                 # GQA: consecutive query heads share a KV head
        K = kc[g, :position + 1].astype(np.float64) * ks[g, :position + 1, None]
        V = vc[g, :position + 1].astype(np.float64) * vs[g, :position + 1, None]
        sc = K @ q[h * hd:(h + 1) * hd].astype(np.float64) / np.sqrt(hd)
        p = np.exp(sc - sc.max())
        want[h] = (p / p.sum()) @ V
    want = want.reshape(-1)
    assert np.linalg.norm(got - want) <= 1e-6 * np.linalg.norm(want)
    if position == 0:
        # one position: softmax weight exactly 1, output = that V row
        assert np.array_equal(got.reshape(nh, hd)[0],
                              np.float32(1.0) * vs[0, 0] * vc[0, 0].astype(np.float32))


# ---- residual add + NaN check ------------------------------------------------
def test_residual_check(oracle):
    res = np.arange(8, dtype=np.float32)
    x = np.ones(8, np.float32)
    out, bad = oracle.residual_check(res, x)
    assert bad == -1 and np.array_equal(out, res + 1)
    x2 = x.copy()
    x2[5] = np.nan
    x2[6] = np.inf
    assert oracle.residual_check(res, x2)[1] == 5
    r3 = np.zeros(4, np.float32)
    edge = np.float32([1e30, -1e30, np.nextafter(np.float32(1e30), np.float32(np.inf)), 0])
    assert oracle.residual_check(r3, edge)[1] == 2          # |v| > 1e30 only


# ---- embedding row: the reference's block dequant ----------------------------
@pytest.mark.parametrize("qt,bs,hd", [(F.Q4, 64, 4096), (F.Q2, 32, 100), (F.Q3, 128, 300),
                                      (F.Q4SYM, 64, 96), (7, 64, 70)])
def test_embed_row_vs_reference_dequant(oracle, ref, qt, bs, hd):
    rng = np.random.default_rng(qt * 10 + hd)
    vocab = 5
    if qt == 7:
        table = F.gaussian(rng, (vocab, hd), 0.02).astype(np.float16).view(np.uint8).reshape(-1)
    else:
        table = np.frombuffer(F.quantize_matrix(F.gaussian(rng, (vocab, hd), 0.02), qt, bs), np.uint8)
    nb = (hd + bs - 1) // bs
    bb = F.block_bytes(qt, bs) if qt != 7 else 0
    for token in (0, 3, vocab - 1):
        got = oracle.embed_row(qt, table, bs, hd, token)
        if qt == 7:
            h = table.view(np.uint16)[token * hd:(token + 1) * hd].copy()
            want = np.empty(hd, np.float32)
            ref.lib.qsf_fp16_to_fp32_array(_p(h), _p(want), hd)
        else:
            want = np.concatenate([
                ref.dequant_block(qt, table[(token * nb + b) * bb:(token * nb + b + 1) * bb],
                                  min(bs, hd - b * bs)) for b in range(nb)])
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
