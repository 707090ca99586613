"""Pin the CPU oracle (oracle/qsf_oracle.c) before trusting it as checker.

Each oracle function is checked against something it did not derive from:
  * golden vectors written by QStream's own compiled C (tests/golden/);
  * the compiled reference itself where oracle/_ref is built (bit-exact);
  * closed forms: IEEE half decoding (numpy), the bit layouts of the packed
    codes (enumerated exhaustively), OCP MX E2M1/E8M0, fp64 brute force.
"""
from __future__ import annotations

import hashlib
import math
import os

import numpy as np
import pytest

from qstream_amd import qsf_format as F

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "qsf_ref_vectors.npz")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def fp16_table(oracle):
    return oracle.fp16_to_fp32_bits(np.arange(65536, dtype=np.uint16))


# ---- fp16 (src/quant.c:11-39) -------------------------------------------------
def test_fp16_all_inputs(oracle, golden):
    table = fp16_table(oracle)
    # golden: digest of the reference's own table over all 65536 inputs
    assert hashlib.sha256(table.tobytes()).digest() == golden["fp16_table_sha256"].tobytes()
    assert np.array_equal(table[golden["fp16_sample_in"]], golden["fp16_sample_out"])
    # closed form: IEEE binary16 (numpy), NaN payload kept as sign|exp|mant<<13
    h = np.arange(65536, dtype=np.uint16)
    ieee = h.view(np.float16).astype(np.float32).view(np.uint32)
    nan = np.isnan(h.view(np.float16))
    assert np.array_equal(table[~nan], ieee[~nan])
    want_nan = ((h[nan].astype(np.uint32) & 0x8000) << 16) | 0x7F800000 | ((h[nan].astype(np.uint32) & 0x3FF) << 13)
    assert np.array_equal(table[nan], want_nan)


# ---- code unpack, enumerated ------------------------------------------------
def test_unpack_2bit_4bit_all_bytes(oracle):
    """Every byte value in every byte position: 2-bit crumbs LSB-first,
    4-bit even index = low nibble (src/quant.c:104-108, 145-152)."""
    for qt, bits in ((F.Q2, 2), (F.Q4, 4), (F.Q4SYM, 4)):
        bs = 256
        per = 8 // bits
        bb = F.block_bytes(qt, bs)
        n = 256
        blocks = np.zeros((n, bb), np.uint8)
        for b in range(n):
            blocks[b, 4:] = (np.arange(bb - 4) + b) % 256
        codes = oracle.unpack_codes_many(qt, blocks, n, bs).astype(np.int32)
        byte = blocks[:, 4:].astype(np.int32)
        want = np.stack([(byte >> (bits * j)) & ((1 << bits) - 1) for j in range(per)], axis=-1).reshape(n, bs)
        if qt == F.Q4SYM:
            want = np.where(want >= 8, want - 16, want)   # two's complement nibble
        assert np.array_equal(codes, want)


def test_unpack_3bit_all_groups(oracle):
    """All 2^24 three-byte groups: code j of a group = (g >> 3j) & 7 with g
    the little-endian 24-bit value (src/quant.c:123-131)."""
    bs = 256                       # 32 groups of 3 bytes per block
    g = np.arange(1 << 24, dtype=np.uint32)
    n = (1 << 24) // 32
    packed = np.stack([(g >> 0) & 0xFF, (g >> 8) & 0xFF, (g >> 16) & 0xFF], axis=-1).astype(np.uint8)
    blocks = np.zeros((n, 4 + 96), np.uint8)
    blocks[:, 4:] = packed.reshape(n, 96)
    codes = oracle.unpack_codes_many(F.Q3, blocks, n, bs)
    want = np.stack([(g >> (3 * j)) & 7 for j in range(8)], axis=-1).astype(np.int8).reshape(n, bs)
    assert np.array_equal(codes, want)


def test_dequant_matches_reference_vectors(oracle, golden):
    for qt in (F.Q2, F.Q3, F.Q4, F.Q4SYM):
        for bs in (32, 64, 128, 256):
            raw = golden[f"deq_q{qt}_bs{bs}_in"]
            want = golden[f"deq_q{qt}_bs{bs}_out"]
            got = np.stack([oracle.dequant_block(qt, raw[i], bs) for i in range(len(raw))])
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (qt, bs)


def test_dequant_closed_form(oracle):
    """v = fp16(scale)*q + fp16(zero), each op rounded to fp32 (asym);
    v = fp16(scale)*q (sym, bytes 2-3 ignored)."""
    rng = np.random.default_rng(9)
    for qt in (F.Q2, F.Q3, F.Q4, F.Q4SYM):
        bs = 64
        raw = rng.integers(0, 256, size=(50, F.block_bytes(qt, bs)), dtype=np.uint8)
        raw[:, 0:4] = rng.standard_normal((50, 2)).astype(np.float16).view(np.uint8).reshape(50, 4)
        codes = oracle.unpack_codes_many(qt, raw, 50, bs).astype(np.float32)
        s = raw[:, 0:2].copy().view(np.float16).astype(np.float32)
        z = raw[:, 2:4].copy().view(np.float16).astype(np.float32)
        want = (s * codes) if qt == F.Q4SYM else (s * codes) + z
        got = np.stack([oracle.dequant_block(qt, raw[i], bs) for i in range(50)])
        assert np.array_equal(got, want.astype(np.float32))


# ---- matvec ------------------------------------------------------------------
def test_matvec_reference_vectors(oracle, golden):
    """72 seeded cases (all types, bs 32..256, partial blocks, outliers):
    bit-exact with the reference's strict scalar outputs."""
    for name in golden["mv_cases"]:
        qt, rows, cols, bs = (int(v) for v in golden[name + "_meta"])
        y = oracle.matvec(qt, golden[name + "_w"], golden[name + "_x"], rows, cols, bs)
        assert np.array_equal(y.view(np.uint32), golden[name + "_y"].view(np.uint32)), name


def test_ramp_vectors(oracle, golden):
    """tests/test_core.c:597-677 (reference quantiser + scalar matvec)."""
    for qt in (F.Q4, F.Q2):
        y = oracle.matvec(qt, golden[f"ramp_q{qt}_w"], golden[f"ramp_q{qt}_x"], 4, 64, 64)
        assert np.array_equal(y, golden[f"ramp_q{qt}_y"])


def _dequant_matrix(oracle, qt, payload, rows, cols, bs):
    base = {F.Q2_OUTLIER: F.Q2, F.Q4_OUTLIER: F.Q4}.get(qt, qt)
    p = np.frombuffer(payload, np.uint8)
    n = 0
    if qt in (F.Q2_OUTLIER, F.Q4_OUTLIER):
        n = int(p[:4].view(np.uint32)[0])
        p = p[4 + 6 * n:]
    nb = (cols + bs - 1) // bs
    bb = F.block_bytes(base, bs)
    W = np.zeros((rows, nb * bs), np.float64)
    for r in range(rows):
        for b in range(nb):
            W[r, b * bs:(b + 1) * bs] = oracle.dequant_block(base, p[(r * nb + b) * bb:], bs)
    return W[:, :cols], n


def test_matvec_fp64_brute_force(oracle):
    """Matvec = dense fp64 product of the dequantised matrix, plus the
    additive fp16 outlier terms (src/quant.c:423-444), to fp32 rounding."""
    rng = np.random.default_rng(17)
    for qt in (F.Q2, F.Q3, F.Q4, F.Q4SYM, F.Q2_OUTLIER, F.Q4_OUTLIER):
        for bs, (rows, cols) in ((64, (12, 256)), (128, (7, 300)), (32, (5, 45))):
            w = F.gaussian(rng, (rows, cols), 0.02)
            x = F.gaussian(rng, cols)
            payload = F.quantize_matrix(w, qt, bs, 0.03)
            W, n = _dequant_matrix(oracle, qt, payload, rows, cols, bs)
            want = W @ x.astype(np.float64)
            if n:
                ent = np.frombuffer(payload, np.uint8)[4:4 + 6 * n].copy().view([("i", "<u4"), ("v", "<u2")])
                for i, v in zip(ent["i"], ent["v"]):
                    r, c = divmod(int(i), cols)
                    if r < rows:
                        want[r] += float(np.uint16(v).view(np.float16)) * float(x[c])
            got = oracle.matvec(qt, payload, x, rows, cols, bs)
            assert np.allclose(got, want, rtol=1e-5, atol=1e-5), (qt, bs)


def test_outlier_rules(oracle):
    """Additive, out-of-range skipped, duplicates twice, n=0 = base matvec."""
    rows, cols, bs = 3, 64, 64
    blocks = bytes(F.quantize_blocks(np.zeros((rows, 64), np.float32), F.Q4).tobytes())
    x = np.arange(cols, dtype=np.float32)
    one = np.float16(1.0).view(np.uint16)
    p = F.outlier_payload([5, 5, rows * cols, 64 + 2], [one, one, one, one], blocks)
    y = oracle.matvec(F.Q4_OUTLIER, p, x, rows, cols, bs)
    assert list(y) == [10.0, 2.0, 0.0]
    p0 = F.outlier_payload([], [], blocks)
    assert list(oracle.matvec(F.Q4_OUTLIER, p0, x, rows, cols, bs)) == [0.0, 0.0, 0.0]


def test_oracle_equals_compiled_reference(oracle, ref):
    """Where the reference tree is present: random cases, bit-exact."""
    rng = np.random.default_rng(23)
    for qt in (F.Q2, F.Q3, F.Q4, F.Q4SYM, F.Q2_OUTLIER, F.Q4_OUTLIER):
        for bs in (32, 64, 128, 256):
            rows, cols = int(rng.integers(1, 20)), int(rng.integers(1, 700))
            w = F.gaussian(rng, (rows, cols), 0.02)
            x = F.gaussian(rng, cols)
            p = F.quantize_matrix(w, qt, bs)
            a = oracle.matvec(qt, p, x, rows, cols, bs)
            b = ref.matvec(qt, p, x, rows, cols, bs)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (qt, bs, rows, cols)
    assert np.array_equal(fp16_table(oracle), ref.fp16_table())


# ---- MXFP4 (OCP MX v1.0) ------------------------------------------------------
def test_e2m1_closed_form(oracle):
    for code in range(16):
        s, e, m = code >> 3, (code >> 1) & 3, code & 1
        mag = m * 0.5 if e == 0 else 2.0 ** (e - 1) * (1 + m / 2)
        want = -mag if s else mag
        got = oracle.lib.orc_e2m1_to_fp32(code)
        assert got == want and math.copysign(1, got) == math.copysign(1, want) or (mag == 0 and got == 0)
    # the converter's LUT (tools/convert_hf.py:1472-1475)
    lut = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]
    assert [oracle.lib.orc_e2m1_to_fp32(c) for c in range(16)] == lut


def test_e8m0_closed_form(oracle):
    for e in range(255):
        assert oracle.lib.orc_e8m0_to_fp32(e) == np.float32(math.ldexp(1.0, e - 127))
    assert math.isnan(oracle.lib.orc_e8m0_to_fp32(255))


def test_mxfp4_matvec_brute_force(oracle):
    rng = np.random.default_rng(31)
    rows, cols = 9, 200
    p = F.random_mxfp4(rng, rows, cols, 100, 140)
    x = F.gaussian(rng, cols)
    nb = (cols + 31) // 32
    buf = np.frombuffer(p, np.uint8)
    codes = buf[:rows * nb * 16].reshape(rows, nb, 16)
    scales = buf[rows * nb * 16:].reshape(rows, nb)
    lut = np.array([oracle.lib.orc_e2m1_to_fp32(c) for c in range(16)])
    W = np.zeros((rows, nb * 32))
    for r in range(rows):
        for b in range(nb):
            for j in range(32):
                nib = (codes[r, b, j // 2] >> (4 * (j % 2))) & 15
                W[r, 32 * b + j] = lut[nib] * 2.0 ** (int(scales[r, b]) - 127)
    want = W[:, :cols] @ x.astype(np.float64)
    got = oracle.matvec(F.MXFP4, p, x, rows, cols, 32)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6 * np.abs(want).max())


# ---- MoE routing (src/engine.c:951-1107) ------------------------------------
def test_topk_reference_case(oracle):
    """tests/test_core.c:712-748: logits {0.1,0.8,0.4,0.6}, top-2 -> 1, 3."""
    idx, w = oracle.topk(np.array([0.1, 0.8, 0.4, 0.6], np.float32), 2, 0)
    assert list(idx) == [1, 3] and np.allclose(w, [0.8, 0.6])


def test_topk_and_softmax_closed_form(oracle):
    rng = np.random.default_rng(5)
    for _ in range(200):
        n, k = int(rng.integers(2, 40)), int(rng.integers(1, 8))
        logits = rng.standard_normal(n).astype(np.float32)
        if rng.random() < 0.3:
            logits[rng.integers(0, n, 3)] = logits[0]          # ties
        p = oracle.softmax(logits)
        e = np.exp(logits.astype(np.float64) - logits.max())
        assert np.allclose(p, e / e.sum(), rtol=1e-6, atol=1e-7)
        order = sorted(range(n), key=lambda i: (-p[i], i))     # ties: lower id first
        kk = min(k, n)
        idx, w = oracle.topk(p, k, 1)
        assert list(idx[:kk]) == order[:kk]
        sel = p[order[:kk]].astype(np.float64)
        if k <= n:
            assert np.allclose(w, sel / sel.sum(), rtol=1e-6)


def test_moe_token_fp64(oracle):
    """One token through the MoE block vs a float64 restatement."""
    rng = np.random.default_rng(8)
    n_exp, k, hidden, eid = 6, 2, 64, 96
    ex = []
    mats = []
    for _ in range(n_exp):
        g, u, d = (F.gaussian(rng, s, 0.05) for s in ((eid, hidden), (eid, hidden), (hidden, eid)))
        pe = {"gate": F.quantize_mxfp4(g), "up": F.quantize_mxfp4(u), "down": F.quantize_mxfp4(d),
              "gate_bias": F.gaussian(rng, eid, 0.1).astype(np.float16).view(np.uint16),
              "up_bias": F.gaussian(rng, eid, 0.1).astype(np.float16).view(np.uint16),
              "down_bias": F.gaussian(rng, hidden, 0.1).astype(np.float16).view(np.uint16)}
        ex.append(pe)
    x = F.gaussian(rng, hidden)
    logits = F.gaussian(rng, n_exp)
    got = oracle.moe_token(ex, k, 1, 2, hidden, eid, x, logits)

    def mv(p, v, r, c):
        return oracle.matvec(F.MXFP4, p, v.astype(np.float32), r, c, 32).astype(np.float64)
    pr = np.exp(logits - logits.max()); pr /= pr.sum()
    top = sorted(range(n_exp), key=lambda i: (-pr[i], i))[:k]
    wts = pr[top] / pr[top].sum()
    want = np.zeros(hidden)
    for wi, e in zip(wts, top):
        f16 = lambda b: b.view(np.float16).astype(np.float64)
        gv = mv(ex[e]["gate"], x, eid, hidden) + f16(ex[e]["gate_bias"])
        uv = mv(ex[e]["up"], x, eid, hidden) + f16(ex[e]["up_bias"])
        h = gv / (1 + np.exp(-gv)) * uv
        want += wi * (mv(ex[e]["down"], h, hidden, eid) + f16(ex[e]["down_bias"]))
    assert np.allclose(got, want, rtol=1e-4, atol=1e-5)


def test_activations(oracle):
    v = np.linspace(-6, 6, 101).astype(np.float32)
    assert np.allclose(oracle.act(2, v), v / (1 + np.exp(-v.astype(np.float64))), rtol=1e-6, atol=1e-7)
    gelu = 0.5 * v * (1 + np.tanh(0.7978845608 * (v + 0.044715 * v.astype(np.float64) ** 3)))
    assert np.allclose(oracle.act(0, v), gelu, rtol=1e-5, atol=1e-6)
    assert np.array_equal(oracle.act(3, v), np.maximum(v, 0))


@pytest.mark.parametrize("m,n,k,bs", [(3, 20, 128, 64), (2, 7, 200, 64), (2, 9, 384, 256)])
def test_prefill_oracle_is_token_loop(oracle, m, n, k, bs):
    """The prefill oracle (weights dequantised once, rows interleaved) equals
    M calls of the scalar matvec bit for bit, odd row counts and partial
    blocks included."""
    rng = np.random.default_rng(4 + n)
    p = F.quantize_matrix(F.gaussian(rng, (n, k), 0.02), F.Q4, bs)
    xb = F.bf16_bits(F.gaussian(rng, (m, k)))
    y = oracle.prefill_4bit(p, xb, m, n, k, bs)
    for t in range(m):
        xf = (xb[t].astype(np.uint32) << 16).view(np.float32)
        assert np.array_equal(y[t], oracle.matvec(F.Q4, p, xf, n, k, bs))


def test_e2m1_encoder_matches_brute_force():
    """qsf_format's threshold E2M1 encoder equals nearest-value rounding with
    ties to the even code, saturating at 6 (OCP MX v1.0), on random values,
    every rounding boundary and its neighbours, and specials."""
    rng = np.random.default_rng(17)
    edges = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], np.float32)
    v = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 3, edges, -edges,
                        np.nextafter(edges, np.float32(0)), np.nextafter(edges, np.float32(10)),
                        np.float32([0.0, -0.0, 6.0, 7.0, 100.0, -100.0, np.inf, -np.inf])])
    mags = F.E2M1_MAG.astype(np.float64)
    mag = np.minimum(np.abs(v.astype(np.float64)), 6.0)
    d = np.abs(mags[None, :] - mag[:, None])
    best = d == d.min(axis=1, keepdims=True)
    even = best & (np.arange(8)[None, :] % 2 == 0)
    idx = np.where(even.any(axis=1), even.argmax(axis=1), best.argmax(axis=1)).astype(np.uint8)
    want = idx | ((np.signbit(v) & (idx != 0)).astype(np.uint8) << 3)
    assert np.array_equal(F._e2m1_encode(v), want)


def test_nonfinite_meta_matches_compiled_reference(oracle, ref):
    """Blocks with Inf or NaN fp16 scale or zero: the oracle's rows equal
    the compiled reference's bit for bit (NaN where Inf * 0 or Inf - Inf
    occurs, the Inf's sign otherwise), and only the poisoned rows go
    non-finite."""
    from tests import meta_cases as MC
    rng = np.random.default_rng(29)
    rows, cols = 24, 700
    for qt in (F.Q2, F.Q3, F.Q4, F.Q4SYM, F.Q2_OUTLIER, F.Q4_OUTLIER):
        for bs in (64, 128):
            p = MC.poison(F.quantize_matrix(F.gaussian(rng, (rows, cols), 0.02), qt, bs), qt, rows, cols, bs)
            x = F.gaussian(rng, cols)
            a = oracle.matvec(qt, p, x, rows, cols, bs)
            b = ref.matvec(qt, p, x, rows, cols, bs)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (qt, bs)
            bad = MC.poisoned_rows(qt, rows, cols, bs)
            assert np.all(~np.isfinite(a[bad])) and np.all(np.isfinite(a[~bad])), (qt, bs)
