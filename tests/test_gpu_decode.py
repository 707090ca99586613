"""GPU parity of the decode GEMV family against the CPU oracle.

Every case calls libqsf_hip through its C ABI (ctypes) on cuda:0 and compares
with oracle/ (a strict restatement of src/kernels_scalar.c and src/quant.c,
itself pinned bit-exactly to the compiled reference in test_oracle.py):
  * unpack: codes, block meta and dequantised values bit-exact;
  * matvec: relative L2 error <= 1e-5 (the tolerance the path is held to), fp32 accumulate.
"""
from __future__ import annotations

import numpy as np
import pytest

from qstream_amd import qsf_format as F
from tests.gpu_util import ENGINES, REL_L2, dev, engine_hip, host, rel_l2, torch_cuda

pytestmark = pytest.mark.gpu

DENSE = [F.Q2, F.Q3, F.Q4, F.Q4SYM]
ALL = DENSE + [F.Q2_OUTLIER, F.Q4_OUTLIER]


@pytest.fixture(scope="module", params=ENGINES, ids=lambda e: f"engine{e}")
def hip(request):
    yield from engine_hip(request)


def _stream():
    return torch_cuda().cuda.current_stream()


def _random_blocks(rng, qt, bs, nblocks, special=False):
    bb = F.block_bytes(qt, bs)
    raw = rng.integers(0, 256, size=(nblocks, bb), dtype=np.uint8)
    # finite fp16 scale/zero, including subnormals, negatives and large values
    s = rng.standard_normal(nblocks).astype(np.float32) * np.float32(0.05)
    z = rng.standard_normal(nblocks).astype(np.float32)
    if special:
        s[::7] = np.float32(3e-6)      # fp16 subnormal
        z[1::5] = np.float32(-6e4)
    raw[:, 0:2] = s.astype(np.float16).view(np.uint8).reshape(-1, 2)
    raw[:, 2:4] = z.astype(np.float16).view(np.uint8).reshape(-1, 2)
    return raw


@pytest.mark.parametrize("qt", DENSE)
@pytest.mark.parametrize("bs", [32, 64, 128, 256])
def test_unpack_bit_exact(hip, oracle, qt, bs):
    """Codes, meta words and dequantised values match src/quant.c:95-177."""
    torch = torch_cuda()
    rng = np.random.default_rng(1000 + 10 * qt + bs)
    n = 97
    raw = _random_blocks(rng, qt, bs, n, special=True)
    d_raw = dev(raw.reshape(-1))
    codes = torch.empty(n * bs, dtype=torch.int8, device="cuda:0")
    meta = torch.empty(n, dtype=torch.int32, device="cuda:0")
    deq = torch.empty(n * bs, dtype=torch.float32, device="cuda:0")
    hip.unpack(qt, d_raw, n, bs, codes, meta, deq, stream=_stream())
    c, m, d = host(codes).reshape(n, bs), host(meta).view(np.uint32), host(deq).reshape(n, bs)
    for b in range(n):
        ref_codes = oracle.unpack_codes(qt, raw[b], bs)
        assert np.array_equal(c[b], ref_codes), f"codes differ in block {b}"
        ref_deq = oracle.dequant_block(qt, raw[b], bs)
        assert np.array_equal(d[b].view(np.uint32), ref_deq.view(np.uint32)), f"dequant differs in block {b}"
    assert np.array_equal(m, raw[:, :4].copy().view(np.uint32).reshape(-1))


def _slots(qt, bs):
    """(w, c, m) -> (code, shift) of the digit tables: which x element (and
    power of two) nibble m of copy c of code dword w is paired with."""
    bits = {F.Q2: 2, F.Q3: 3}.get(qt, 4)
    cw, nc = bs * bits // 32, (2 if bits in (2, 3) else 1)
    out = {}
    for w in range(cw):
        for c in range(nc):
            for m in range(8):
                if bits == 2:
                    out[w, c, m] = (16 * w + 2 * m + c, 0)
                elif bits == 3:
                    g = 8 * w + m
                    out[w, c, m] = ((4 * g) // 3 + c, g % 3)
                else:
                    out[w, c, m] = (8 * w + m, 0)
    return cw, nc, out


@pytest.mark.parametrize("qt,bs", [(F.Q4, 64), (F.Q2, 64), (F.Q3, 128), (F.Q4SYM, 32),
                                   (F.Q3, 32), (F.Q2, 256), (F.Q4, 256)])
def test_xprep_digits_exact(hip, qt, bs):
    """x -> block-fixed-point X = rint(x * 2^sh) with amax * 2^sh < 2^XB, and
    the six balanced base-16 digit words of every multiplier X * 2^shift,
    reconstructed exactly; block meta f = 2^-sh and sum(X) * f in fp32.
    Blocks of 128 or 256 codes are prepared per 64-code part (the unit the
    split GEMV reads them in), so their digits are those of 64-code blocks."""
    torch = torch_cuda()
    rng = np.random.default_rng(bs + qt)
    stored = bs
    cols = 5 * stored + stored // 2 + 3          # partial last block
    x = F.gaussian(rng, cols)
    x[stored:2 * stored] = 0.0                   # an all-zero block
    x[2 * stored:3 * stored] *= np.float32(1e-30)    # tiny scale
    x[3 * stored:4 * stored] *= np.float32(2.0 ** 120)   # huge scale (negative shift)
    bs = min(bs, 64)                             # the prepared unit
    nb = (cols + bs - 1) // bs
    cw, nc, slots = _slots(qt, bs)
    nd = 6
    dw = cw * nc * nd                            # digit words a block, a multiple of 4
    dws = dw if (dw // 4) % 2 else dw + 4        # stride: an odd number of 16-byte quads
    xb = 20 if qt == F.Q3 else 22
    nbytes = hip.xprep_bytes(qt, stored, cols)
    assert nbytes == hip.xprep_bytes(qt, bs, cols)
    buf = torch.zeros(nbytes + 256, dtype=torch.uint8, device="cuda:0")
    addr = (buf.data_ptr() + 255) & ~255
    hip.xprep(qt, stored, cols, dev(x), addr, stream=_stream())
    raw = host(buf)[addr - buf.data_ptr():][:nbytes]
    dig = raw[:nb * dws * 4].view(np.uint32).reshape(nb, dws)
    moff = (nb * dws * 4 + 255) & ~255
    meta = raw[moff:moff + nb * 8].view(np.float32).reshape(nb, 2)
    xp = np.zeros(nb * bs, np.float64)
    xp[:cols] = x
    for b in range(nb):
        blk = xp[b * bs:(b + 1) * bs]
        amax = np.abs(blk).max()
        sh = 0 if amax == 0 else xb - 1 - int(np.floor(np.log2(amax)))
        sh = min(sh, 126)
        X = np.rint(blk * 2.0 ** sh).astype(np.int64)
        assert np.abs(X).max() <= 2 ** xb
        # meta = {2^-sh exactly, 2^-sh * sum X rounded once to fp32}
        assert meta[b, 0] == np.float32(2.0 ** -sh), (b, meta[b, 0], sh)
        assert meta[b, 1] == np.float32(float(X.sum()) * 2.0 ** -sh), (b, meta[b, 1])
        for (w, c, m), (code, shift) in slots.items():
            words = dig[b, (w * nc + c) * nd:(w * nc + c) * nd + nd]
            nib = (words >> np.uint32(4 * m)) & np.uint32(15)
            sd = np.where(nib >= 8, nib.astype(np.int64) - 16, nib.astype(np.int64))
            rec = int(sum(int(sd[d]) * 16 ** d for d in range(nd)))
            assert rec == int(X[code]) * 2 ** shift, (b, w, c, m, rec, X[code])


def _case(oracle, qt, rows, cols, bs, seed, outlier_frac=0.005):
    rng = np.random.default_rng(seed)
    w = F.gaussian(rng, (rows, cols), 0.02)
    x = F.gaussian(rng, cols)
    payload = F.quantize_matrix(w, qt, bs, outlier_frac)
    ref = oracle.matvec(qt, payload, x, rows, cols, bs)
    return payload, x, ref


SHAPES = [(64, 64), (37, 300), (5, 33), (130, 1000), (300, 4096), (1, 17), (96, 2880)]


@pytest.mark.parametrize("qt", ALL)
@pytest.mark.parametrize("bs", [32, 64, 128, 256])
def test_matvec_slot_parity(hip, oracle, qt, bs):
    """Drop-in table slot (host pointers, synchronous) vs scalar oracle."""
    kt = hip.KernelTable()
    slot = {F.Q2: kt.matvec_2bit, F.Q3: kt.matvec_3bit, F.Q4: kt.matvec_4bit,
            F.Q4SYM: kt.matvec_4bit_sym, F.Q2_OUTLIER: kt.matvec_outlier_2bit,
            F.Q4_OUTLIER: kt.matvec_outlier_4bit}[qt]
    for i, (rows, cols) in enumerate(SHAPES):
        payload, x, ref = _case(oracle, qt, rows, cols, bs, seed=7 * i + qt * 131 + bs)
        out = np.full(rows, np.nan, np.float32)
        slot(payload, x, out, rows, cols, bs)
        err = rel_l2(out, ref)
        print(f"qt={qt} bs={bs} {rows}x{cols} rel_l2={err:.3e}")
        assert err <= REL_L2, (qt, bs, rows, cols, err)


def test_reference_ramp_cases(hip, oracle):
    """tests/test_core.c:597-677: 4x64 ramp, 4-bit and 2-bit, through the slots."""
    rows, cols, bs = 4, 64, 64
    w = (np.arange(rows * cols, dtype=np.float32) / 256.0 - 0.5).reshape(rows, cols)
    x = np.arange(cols, dtype=np.float32) / 64.0 - 0.5
    kt = hip.KernelTable()
    for qt, slot in ((F.Q4, kt.matvec_4bit), (F.Q2, kt.matvec_2bit)):
        payload = F.quantize_matrix(w, qt, bs)
        ref = oracle.matvec(qt, payload, x, rows, cols, bs)
        out = np.zeros(rows, np.float32)
        slot(payload, x, out, rows, cols, bs)
        assert np.max(np.abs(out - ref)) <= 1e-3
        assert rel_l2(out, ref) <= REL_L2


@pytest.mark.parametrize("qt,rows,cols,bs", [
    (F.Q4, 4096, 4096, 64),              # config 0
    (F.Q2_OUTLIER, 11008, 4096, 64),     # config 1 (one of gate/up)
    (F.Q3, 4096, 11008, 128),            # config 2 down_proj
    (F.Q3, 11008, 4096, 128),            # config 2 gate/up
    (F.Q3, 70, 16384, 128),              # digits exceed LDS: K in chunks
    (F.Q4, 37, 20000, 64),               # K in chunks, partial last block
])
def test_matvec_full_shapes(hip, oracle, qt, rows, cols, bs):
    torch = torch_cuda()
    rng = np.random.default_rng(rows + cols + qt)
    if qt == F.Q2_OUTLIER:
        w = F.heavy_tail_weights(rng, rows, cols)
    else:
        w = F.gaussian(rng, (rows, cols), 0.02)
    x = F.gaussian(rng, cols)
    payload = F.quantize_matrix(w, qt, bs)
    ref = oracle.matvec(qt, payload, x, rows, cols, bs)
    t = hip.Tensor(payload, qt, rows, cols, bs)
    y = torch.full((rows,), float("nan"), device="cuda:0")
    t.matvec(dev(x), y, stream=_stream())
    err = rel_l2(host(y), ref)
    print(f"full qt={qt} {rows}x{cols} bs{bs}: rel_l2={err:.3e}")
    assert err <= REL_L2
    t.free()


def test_group_launch_matches_single(hip, oracle):
    """gate+up in one launch equals two single launches (and the oracle)."""
    torch = torch_cuda()
    rng = np.random.default_rng(5)
    rows, cols, bs = 1100, 4096, 64
    ts, refs = [], []
    x = F.gaussian(rng, cols)
    for r in (rows, rows + 7):
        w = F.heavy_tail_weights(rng, r, cols)
        p = F.quantize_matrix(w, F.Q2_OUTLIER, bs)
        ts.append(hip.Tensor(p, F.Q2_OUTLIER, r, cols, bs))
        refs.append(oracle.matvec(F.Q2_OUTLIER, p, x, r, cols, bs))
    dx = dev(x)
    ys = [torch.empty(t.rows, device="cuda:0") for t in ts]
    hip.matvec_group(ts, dx, ys, stream=_stream())
    singles = [torch.empty(t.rows, device="cuda:0") for t in ts]
    for t, y in zip(ts, singles):
        t.matvec(dx, y, stream=_stream())
    for y, s, ref in zip(ys, singles, refs):
        assert np.array_equal(host(y), host(s))
        assert rel_l2(host(y), ref) <= REL_L2


def test_outlier_edge_cases(hip, oracle):
    """Out-of-range entries are skipped, duplicates add twice, n=0 is plain
    (src/quant.c:423-444)."""
    rows, cols, bs = 9, 128, 64
    rng = np.random.default_rng(11)
    w = F.gaussian(rng, (rows, cols), 0.02)
    x = F.gaussian(rng, cols)
    blocks = F.quantize_blocks(F._row_blocks(w, bs), F.Q2).tobytes()
    vals = np.array([1.5, -2.0, 0.75, 3.0, 1.0, -1.0], np.float16).view(np.uint16)
    idx = np.array([5, rows * cols + 3, 5, 0, rows * cols - 1, 2 * rows * cols], np.uint32)
    kt = hip.KernelTable()
    for n in (0, len(idx)):
        payload = F.outlier_payload(idx[:n], vals[:n], blocks)
        ref = oracle.matvec(F.Q2_OUTLIER, payload, x, rows, cols, bs)
        out = np.zeros(rows, np.float32)
        kt.matvec_outlier_2bit(payload, x, out, rows, cols, bs)
        assert rel_l2(out, ref) <= REL_L2, n


@pytest.mark.parametrize("qt", ALL)
def test_constant_x_large_blocks(hip, oracle, qt):
    """Same-sign x fills a 256-code block with |X| near 2^XB: the block sum of
    X reaches 2^30 and must not wrap."""
    rows, cols, bs = 33, 1000, 256
    rng = np.random.default_rng(qt + 40)
    w = F.gaussian(rng, (rows, cols), 0.02)
    payload = F.quantize_matrix(w, qt, bs)
    for x in (np.ones(cols, np.float32), np.full(cols, -3.0e-3, np.float32)):
        ref = oracle.matvec(qt, payload, x, rows, cols, bs)
        out = np.full(rows, np.nan, np.float32)
        _slot(hip, qt)(payload, x, out, rows, cols, bs)
        assert rel_l2(out, ref) <= REL_L2, (qt, x[0])


@pytest.mark.parametrize("qt,bs", [(F.Q2, 64), (F.Q3, 128), (F.Q4, 64), (F.Q4SYM, 64),
                                   (F.Q2_OUTLIER, 64), (F.Q4_OUTLIER, 128)])
def test_spiky_activations(hip, oracle, qt, bs):
    """Decoder activations with a few channels 100-1000x the rest: the spike
    sets its block's fixed-point scale, so the block's small entries keep
    fewer bits.  The result must still meet the bar at a 7B shape."""
    rows, cols = 512, 4096
    rng = np.random.default_rng(qt * 7 + bs)
    w = (F.heavy_tail_weights(rng, rows, cols) if qt in (F.Q2_OUTLIER, F.Q4_OUTLIER)
         else F.gaussian(rng, (rows, cols), 0.02))
    payload = F.quantize_matrix(w, qt, bs)
    x = F.gaussian(rng, cols)
    spikes = rng.choice(cols, 24, replace=False)
    x[spikes] *= rng.uniform(100.0, 1000.0, 24).astype(np.float32)
    ref = oracle.matvec(qt, payload, x, rows, cols, bs)
    out = np.full(rows, np.nan, np.float32)
    _slot(hip, qt)(payload, x, out, rows, cols, bs)
    err = rel_l2(out, ref)
    print(f"spiky x qt={qt} bs={bs}: rel_l2 = {err:.3e}")
    assert err <= REL_L2, err


@pytest.mark.parametrize("qt", [F.Q2_OUTLIER, F.Q4_OUTLIER])
@pytest.mark.parametrize("rows,cols,bs,frac", [
    (40, 4096, 64, 0.2),       # ~800 entries a row: many steps of the sparse pass
    (70, 300, 32, 0.3),        # 16-lane row groups, ~90 entries a row
    (3, 70000, 64, 0.01),      # columns beyond 16 bits: split entry tables
])
def test_outlier_dense_and_wide(hip, oracle, qt, rows, cols, bs, frac):
    rng = np.random.default_rng(rows * 7 + qt)
    x = F.gaussian(rng, cols)
    w = F.gaussian(rng, (rows, cols), 0.02)
    payload = F.quantize_matrix(w, qt, bs, frac)
    ref = oracle.matvec(qt, payload, x, rows, cols, bs)
    out = np.full(rows, np.nan, np.float32)
    _slot(hip, qt)(payload, x, out, rows, cols, bs)
    err = rel_l2(out, ref)
    print(f"outlier qt={qt} {rows}x{cols} frac={frac}: rel_l2={err:.3e}")
    assert err <= REL_L2


def test_outlier_many_short_rows(hip, oracle):
    """1.6M rows of one block: 128-row tiles, the per-wave result stash caps
    the tiles a workgroup takes."""
    rows, cols, bs = 1_600_000, 17, 32
    rng = np.random.default_rng(99)
    w = F.gaussian(rng, (rows, cols), 0.02)
    x = F.gaussian(rng, cols)
    payload = F.quantize_matrix(w, F.Q2_OUTLIER, bs)
    del w
    ref = oracle.matvec(F.Q2_OUTLIER, payload, x, rows, cols, bs)
    torch = torch_cuda()
    t = hip.Tensor(payload, F.Q2_OUTLIER, rows, cols, bs)
    y = torch.full((rows,), float("nan"), device="cuda:0")
    t.matvec(dev(x), y, stream=_stream())
    err = rel_l2(host(y), ref)
    t.free()
    assert err <= REL_L2, err


def _slot(hip, qt):
    kt = hip.KernelTable()
    return {F.Q2: kt.matvec_2bit, F.Q3: kt.matvec_3bit, F.Q4: kt.matvec_4bit,
            F.Q4SYM: kt.matvec_4bit_sym, F.Q2_OUTLIER: kt.matvec_outlier_2bit,
            F.Q4_OUTLIER: kt.matvec_outlier_4bit}[qt]


def test_degenerate_shapes(hip, oracle):
    kt = hip.KernelTable()
    # rows = 0: no-op
    out = np.full(3, 7.0, np.float32)
    kt.matvec_4bit(b"\x00" * 64, np.zeros(4, np.float32), out, 0, 4, 64)
    assert np.all(out == 7.0)
    # cols = 0: the scalar reference writes zeros
    out = np.full(5, 7.0, np.float32)
    kt.matvec_4bit(b"\x00" * 64, np.zeros(1, np.float32), out, 5, 0, 64)
    assert np.all(out == 0.0)


@pytest.mark.parametrize("qt", [F.Q2, F.Q3, F.Q4, F.Q4SYM, F.Q2_OUTLIER])
@pytest.mark.parametrize("bad", [np.inf, -np.inf, np.nan])
def test_nonfinite_input_gives_nan(hip, qt, bad):
    """Documented divergence: a non-finite x value makes every output row
    NaN.  The scalar reference gives +-Inf for rows whose weight at that
    column is nonzero (NaN only for 0 * Inf or Inf - Inf); the block
    fixed-point x cannot carry an infinity, so the whole result is marked
    invalid instead, which the engine's NaN check catches
    (src/engine.c:1174-1187)."""
    rows, cols, bs = 8, 256, 64
    rng = np.random.default_rng(3)
    p = F.quantize_matrix(F.heavy_tail_weights(rng, rows, cols), qt, bs)
    x = F.gaussian(rng, cols)
    x[70] = bad
    out = np.zeros(rows, np.float32)
    slot = {F.Q2: "matvec_2bit", F.Q3: "matvec_3bit", F.Q4: "matvec_4bit",
            F.Q4SYM: "matvec_4bit_sym", F.Q2_OUTLIER: "matvec_outlier_2bit"}[qt]
    getattr(hip.KernelTable(), slot)(p, x, out, rows, cols, bs)
    assert np.all(np.isnan(out)), out


@pytest.mark.parametrize("qt", ALL)
@pytest.mark.parametrize("bs", [64, 128])
def test_nonfinite_meta_rows(hip, oracle, qt, bs):
    """Blocks whose fp16 scale or zero is Inf or NaN.  Decided behaviour:
    exactly the rows the reference makes non-finite are non-finite here,
    and every other row keeps the 1e-5 bar.  Which of NaN and +-Inf such a
    row holds can differ: the reference takes Inf * 0 per element
    ((scale * q + zero) * x, src/kernels_scalar.c:16-109), this path
    multiplies the block's sums by scale and zero once."""
    from tests import meta_cases as MC
    torch = torch_cuda()
    rows, cols = 40, 1000
    rng = np.random.default_rng(41 + qt + bs)
    w = F.heavy_tail_weights(rng, rows, cols) if qt in (F.Q2_OUTLIER, F.Q4_OUTLIER) else \
        F.gaussian(rng, (rows, cols), 0.02)
    p = MC.poison(F.quantize_matrix(w, qt, bs), qt, rows, cols, bs)
    x = F.gaussian(rng, cols)
    ref = oracle.matvec(qt, p, x, rows, cols, bs)
    bad = MC.poisoned_rows(qt, rows, cols, bs)
    assert np.all(~np.isfinite(ref[bad])) and np.all(np.isfinite(ref[~bad]))
    print(f"nonfinite meta qt {qt} bs {bs}", flush=True)
    t = hip.Tensor(np.frombuffer(p, np.uint8).copy(), qt, rows, cols, bs)
    try:
        y = torch.full((rows,), 0.5, device="cuda:0")
        t.matvec(dev(x), y, stream=_stream())
        outs = [host(y)]
    finally:
        t.free()
    slot = np.zeros(rows, np.float32)
    getattr(hip.KernelTable(), {F.Q2: "matvec_2bit", F.Q3: "matvec_3bit", F.Q4: "matvec_4bit",
                                 F.Q4SYM: "matvec_4bit_sym", F.Q2_OUTLIER: "matvec_outlier_2bit",
                                 F.Q4_OUTLIER: "matvec_outlier_4bit"}[qt])(p, x, slot, rows, cols, bs)
    outs.append(slot)
    for got in outs:
        assert np.array_equal(~np.isfinite(got), bad), (got, bad)
        assert rel_l2(got[~bad], ref[~bad]) <= REL_L2


def _unsampled_edit(payload: np.ndarray) -> np.ndarray:
    """A copy of `payload` changed in one byte that none of the slot's nine
    sampled 8-byte words covers (offset n/16, inside the first eighth)."""
    n = payload.size
    pos = n // 16
    assert 8 <= pos and pos + 1 < n // 8
    out = payload.copy()
    out[pos] ^= 0x5A
    return out


@pytest.mark.parametrize("qt", [F.Q4, F.Q2_OUTLIER])
def test_slot_reused_buffer_forget_and_volatile(hip, oracle, qt):
    """A reused host buffer (src/engine.c:786-789 decompresses every layer
    into one layer_buf) is never served stale weights when the caller keeps
    the contract: qsf_hip_arena_forget after a rewrite whose first change
    only an unsampled byte shows; and once the slot has seen the content
    change, the pointer is volatile and every rewrite is picked up."""
    rows, cols, bs = 300, 4096, 64
    rng = np.random.default_rng(11 + qt)
    mk = (lambda: F.heavy_tail_weights(rng, rows, cols)) if qt == F.Q2_OUTLIER else \
        (lambda: F.gaussian(rng, (rows, cols), 0.02))
    a = np.frombuffer(F.quantize_matrix(mk(), qt, bs), np.uint8).copy()
    b = _unsampled_edit(a)
    c = np.frombuffer(F.quantize_matrix(mk(), qt, bs), np.uint8).copy()
    assert c.size == a.size
    x = F.gaussian(rng, cols)
    slot = _slot(hip, qt)
    buf = a.copy()
    # a fresh buffer: entries that earlier, freed arrays left at these
    # addresses (this test under another engine wrote the same bytes there)
    # are the caller's to drop
    hip.arena_forget_range(buf)
    out = np.full(rows, np.nan, np.float32)

    def run_and_check(content):
        out[:] = np.nan
        slot(buf, x, out, rows, cols, bs)
        assert rel_l2(out, oracle.matvec(qt, content.tobytes(), x, rows, cols, bs)) <= REL_L2

    run_and_check(a)
    buf[:] = b                                   # first rewrite: only an unsampled byte
    assert hip.arena_forget(buf)                 # the contract
    run_and_check(b)
    assert not np.array_equal(oracle.matvec(qt, a.tobytes(), x, rows, cols, bs),
                              oracle.matvec(qt, b.tobytes(), x, rows, cols, bs))
    buf[:] = c                                   # sampled words change: volatile from now on
    run_and_check(c)
    buf[:] = _unsampled_edit(c)                  # caught without forget: the pointer is volatile
    run_and_check(buf.copy())
    buf[:] = c
    run_and_check(c)
    assert hip.arena_forget(buf) and not hip.arena_forget(buf)
    # the range form, as after an LZ4 layer is decompressed again
    run_and_check(c)
    buf[:] = b
    # >= 1: keys that earlier, freed arrays left inside this address range go too
    assert hip.arena_forget_range(buf) >= 1 and hip.arena_forget_range(buf) == 0
    run_and_check(b)
    hip.arena_forget_range(buf)                  # before the buffer is freed


def test_slot_x_reuse_between_calls(hip, oracle):
    """The slots keep the last call's prepared x in HBM and skip the
    preparation when x is bit-identical and the format, block size and
    length match.  Every change of any of these must be picked up: same x
    across matrices (gate, up), one element changed, another format or block
    size at the same length, a shorter x, and an MXFP4 call in between."""
    rng = np.random.default_rng(21)
    cols = 4096
    cases = [(F.Q2_OUTLIER, 64, 700), (F.Q2_OUTLIER, 64, 500), (F.Q4, 64, 300),
             (F.Q4, 128, 300), (F.Q3, 128, 260), (F.Q4SYM, 32, 130)]
    mats = []
    for qt, bs, rows in cases:
        w = F.heavy_tail_weights(rng, rows, cols) if qt == F.Q2_OUTLIER else \
            F.gaussian(rng, (rows, cols), 0.02)
        mats.append((qt, bs, rows, F.quantize_matrix(w, qt, bs)))
    x = F.gaussian(rng, cols)
    x2 = x.copy()
    x2[1234] += 0.5
    mx = F.quantize_mxfp4(F.gaussian(rng, (64, cols), 0.02))
    kt = hip.KernelTable()

    def check(i, xv):
        qt, bs, rows, p = mats[i]
        out = np.full(rows, np.nan, np.float32)
        _slot(hip, qt)(p, xv.copy(), out, rows, cols, bs)
        assert rel_l2(out, oracle.matvec(qt, p, xv, rows, cols, bs)) <= REL_L2, (i, qt, bs)

    for seq in ([0, 1, 1, 0], [2, 3, 2], [4, 5, 0]):
        for i in seq:
            check(i, x)
    check(0, x2)
    check(1, x2)
    check(1, x)
    out = np.full(64, np.nan, np.float32)
    kt.matvec_mxfp4(mx, x, out, 64, cols, 32)
    assert rel_l2(out, oracle.matvec(F.MXFP4, mx, x, 64, cols, 32)) <= REL_L2
    check(1, x)
    # a shorter x whose leading bytes equal the last one's
    qt, bs, rows, _ = mats[2]
    short = 2048
    p = F.quantize_matrix(F.gaussian(rng, (rows, short), 0.02), qt, bs)
    out = np.full(rows, np.nan, np.float32)
    _slot(hip, qt)(p, x[:short].copy(), out, rows, short, bs)
    assert rel_l2(out, oracle.matvec(qt, p, x[:short], rows, short, bs)) <= REL_L2
    check(2, x)


@pytest.mark.parametrize("qt,bs", [(F.Q2_OUTLIER, 64), (F.Q4_OUTLIER, 64)])
def test_outlier_rows_across_pass_boundaries(hip, oracle, qt, bs):
    """A 64-lane row group takes a row's first 64 outlier entries in one pass
    (one entry a lane) and the rest in further passes.  Rows with 0, 1, 63,
    64, 65, 100, 128 and 129 entries straddle those boundaries, among rows of
    2 or 0; duplicates and an out-of-range entry as usual.  Both the device
    path and the table slot, and every row on its own."""
    torch = torch_cuda()
    rows, cols = 300, 4096
    rng = np.random.default_rng(61 + qt)
    base = F.Q2 if qt == F.Q2_OUTLIER else F.Q4
    counts = {3: 1, 10: 63, 11: 64, 12: 65, 13: 100, 14: 128, 15: 129, 299: 100, 150: 7}
    idx, vals = [], []
    for r in range(rows):
        c = counts.get(r, 2 if r % 5 else 0)
        cs = rng.choice(cols, size=c, replace=False)
        idx += [r * cols + int(k) for k in cs]
        vals += list(rng.standard_normal(c) * 0.5)
    idx += [15 * cols + 7, 15 * cols + 7, rows * cols + 5]      # duplicate pair, out of range
    vals += [1.0, 2.0, 9.0]
    w = F.gaussian(rng, (rows, cols), 0.02)
    blocks = F.quantize_blocks(F._row_blocks(w, bs), base).tobytes()
    payload = F.outlier_payload(np.array(idx, np.uint32),
                                np.array(vals, np.float16).view(np.uint16), blocks)
    x = F.gaussian(rng, cols)
    ref = oracle.matvec(qt, payload, x, rows, cols, bs)
    t = hip.Tensor(payload, qt, rows, cols, bs)
    y = torch.full((rows,), float("nan"), device="cuda:0")
    t.matvec(dev(x), y, stream=_stream())
    assert rel_l2(host(y), ref) <= REL_L2, "device"
    t.free()
    out = np.full(rows, np.nan, np.float32)
    _slot(hip, qt)(payload, x, out, rows, cols, bs)
    assert rel_l2(out, ref) <= REL_L2, "slot"
    np.testing.assert_allclose(out, ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())


@pytest.mark.parametrize("qt", [F.Q2, F.Q3, F.Q4, F.Q4SYM, F.Q2_OUTLIER])
@pytest.mark.parametrize("bs", [128, 256])
@pytest.mark.parametrize("rows,cols", [(300, 4096), (4096, 4096), (512, 11008), (200, 1000), (33, 800)])
def test_split_block_view(hip, oracle, qt, bs, rows, cols):
    """One-launch device calls read 128- and 256-code blocks as 64-code
    parts sharing the stored block's meta when that keeps more lanes of a
    row group busy (few rows, 86 blocks a row); partial last blocks
    included.  Against the oracle, and against the table slot, which runs
    on prepared x at the stored block size."""
    torch = torch_cuda()
    rng = np.random.default_rng(rows + cols + bs + qt)
    w = F.heavy_tail_weights(rng, rows, cols) if qt == F.Q2_OUTLIER else F.gaussian(rng, (rows, cols), 0.02)
    x = F.gaussian(rng, cols)
    payload = F.quantize_matrix(w, qt, bs)
    ref = oracle.matvec(qt, payload, x, rows, cols, bs)
    t = hip.Tensor(payload, qt, rows, cols, bs)
    y = torch.full((rows,), float("nan"), device="cuda:0")
    t.matvec(dev(x), y, stream=_stream())
    got = host(y)
    t.free()
    assert rel_l2(got, ref) <= REL_L2, "device"
    out = np.full(rows, np.nan, np.float32)
    _slot(hip, qt)(payload, x, out, rows, cols, bs)
    assert rel_l2(out, ref) <= REL_L2, "slot"
