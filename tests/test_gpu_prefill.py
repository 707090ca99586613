"""Batched prefill (config 4) on MFMA: Y[m] = W float(bf16 x[m]).

The specification is M token-by-token src/kernels_scalar.c:64-85 matvecs on
float(bf16(x)) (the engine prefills one token at a time,
src/engine.c:1289-1295): oracle.prefill_4bit.  The bar is north_star's
1e-5 rel-L2 against it, on every shape, and at config-4 shape on row slices
of the full launch.  A second reference, fp64 products of the fp32
dequantised weights, shows how far each side is from exact.
"""
import numpy as np
import pytest

from qstream_amd import qsf_format as F
from tests.gpu_util import ENGINES, REL_L2, engine_hip, rel_l2, torch_cuda

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", params=ENGINES, ids=lambda e: f"engine{e}")
def hip(request):
    yield from engine_hip(request)


def bf16_rne(a32: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even (finite inputs)."""
    b = np.ascontiguousarray(a32, np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f64(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def dequant_f64(oracle, payload, n, k, bs) -> np.ndarray:
    """The reference's weights, fp32(s*q + z) (src/quant.c:136-155), as fp64
    [n][k]."""
    nb = (k + bs - 1) // bs
    bb = 4 + bs // 2
    raw = np.frombuffer(payload, np.uint8)[:n * nb * bb]
    q = oracle.unpack_codes_many(F.Q4, raw.tobytes(), n * nb, bs).astype(np.float32)
    meta = raw.reshape(n * nb, bb)[:, :4].copy().view(np.uint16)
    s = oracle.fp16_to_fp32_bits(meta[:, 0]).view(np.float32)[:, None]
    z = oracle.fp16_to_fp32_bits(meta[:, 1]).view(np.float32)[:, None]
    w32 = ((s * q.reshape(n * nb, bs)) + z).astype(np.float32)   # s*q exact; one rounding in +
    return w32.astype(np.float64).reshape(n, nb * bs)[:, :k]


def case(seed, m, n, k, bs=64):
    rng = np.random.default_rng(seed)
    w = F.gaussian(rng, (n, k), 0.02)
    payload = F.quantize_matrix(w, F.Q4, bs)
    xb = bf16_rne(rng.standard_normal((m, k)).astype(np.float32))
    return payload, xb


def run(hip, payload, xb, m, n, k, bs):
    torch = torch_cuda()
    t = hip.Tensor(payload, F.Q4, n, k, bs)
    dx = torch.from_numpy(xb.view(np.int16).copy()).to("cuda:0")
    y = torch.full((m, n), float("nan"), device="cuda:0")
    t.prefill(dx, m, y, stream=torch.cuda.current_stream())
    torch.cuda.synchronize()
    out = y.cpu().numpy()
    t.free()
    return out


def row_slice(payload, r0, r1, k, bs):
    """Payload bytes of rows r0..r1-1 (rows are contiguous runs of blocks)."""
    rb = ((k + bs - 1) // bs) * (4 + bs // 2)
    return bytes(payload[r0 * rb:r1 * rb])


# (m, n, k, bs): single tile, ragged k and partial blocks, several m and n
# tiles, every block size, n and m past a tile edge
# the last two: rows of 448 blocks (the most the zero-point stash holds) and
# of 449, whose zero-point stages read the meta from memory again
SHAPES = [(1, 64, 64, 64), (37, 100, 256, 64), (128, 64, 512, 64), (200, 300, 1000, 64),
          (130, 70, 512, 128), (64, 96, 768, 256), (513, 129, 4096, 64), (16, 112, 200, 128),
          (300, 224, 1280, 256), (24, 120, 28672, 64), (20, 112, 28736, 64)]


@pytest.mark.parametrize("m,n,k,bs", SHAPES)
def test_prefill_vs_scalar_oracle(hip, oracle, m, n, k, bs):
    payload, xb = case(m * 7 + n + k, m, n, k, bs)
    got = run(hip, payload, xb, m, n, k, bs)
    ref = oracle.prefill_4bit(payload, xb, m, n, k, bs)
    err = rel_l2(got, ref)
    exact = bf16_to_f64(xb) @ dequant_f64(oracle, payload, n, k, bs).T
    print(f"prefill {m}x{n}x{k} bs{bs}: rel_l2 vs scalar oracle {err:.3e}, "
          f"vs fp64 {rel_l2(got, exact):.3e} (oracle vs fp64 {rel_l2(ref, exact):.3e})")
    assert np.all(np.isfinite(got))
    assert err <= REL_L2, err


def test_prefill_config4_slices(hip, oracle):
    """Benchmark config 4 (M=512, K=4096, N=14336, block 64) as one launch;
    two 1024-row slices (the first and the last n tiles) against the
    scalar oracle, and every output finite."""
    m, n, k, bs = 512, 14336, 4096, 64
    payload, xb = case(4, m, n, k, bs)
    got = run(hip, payload, xb, m, n, k, bs)
    assert np.all(np.isfinite(got))
    for r0, r1 in ((0, 1024), (n - 1024, n)):
        ref = oracle.prefill_4bit(row_slice(payload, r0, r1, k, bs), xb, m, r1 - r0, k, bs)
        err = rel_l2(got[:, r0:r1], ref)
        print(f"prefill config 4 rows {r0}..{r1}: rel_l2 vs scalar oracle = {err:.3e}")
        assert err <= REL_L2, err


def test_prefill_graph_survives_workspace_growth(hip, oracle):
    """A graph captured at small m keeps its workspace address: a later,
    larger eager call that grows the library workspace must not free it.
    Each replay (with eager work and a synchronisation between) matches the
    oracle."""
    torch = torch_cuda()
    n, k, bs = 128, 512, 64
    small, big = 16, 512
    payload, xb = case(11, big, n, k, bs)
    t = hip.Tensor(payload, F.Q4, n, k, bs)
    dx = torch.from_numpy(xb.view(np.int16).copy()).to("cuda:0")
    y_small = torch.full((small, n), float("nan"), device="cuda:0")
    y_big = torch.full((big, n), float("nan"), device="cuda:0")
    ref = oracle.prefill_4bit(payload, xb, big, n, k, bs)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        t.prefill(dx, small, y_small, stream=stream)        # sizes the workspace
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        t.prefill(dx, small, y_small, stream=stream)
    torch.cuda.synchronize()
    t.prefill(dx, big, y_big, stream=torch.cuda.current_stream())   # grows it
    torch.cuda.synchronize()
    assert rel_l2(y_big.cpu().numpy(), ref) <= REL_L2
    for rep in range(3):
        y_small.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        err = rel_l2(y_small.cpu().numpy(), ref[:small])
        print(f"replay {rep}: rel_l2 {err:.3e}")
        assert err <= REL_L2, err
    del g
    t.free()


def test_prefill_rejects_bad_input(hip):
    torch = torch_cuda()
    rng = np.random.default_rng(0)
    t2 = hip.Tensor(F.quantize_matrix(F.gaussian(rng, (8, 64), 0.02), F.Q2, 64), F.Q2, 8, 64, 64)
    x = torch.zeros((4, 64), dtype=torch.int16, device="cuda:0")
    y = torch.zeros((4, 8), device="cuda:0")
    with pytest.raises(hip.QsfHipError):
        t2.prefill(x, 4, y)                     # not a 4-bit tensor
    t2.free()
    t4 = hip.Tensor(F.quantize_matrix(F.gaussian(rng, (8, 64), 0.02), F.Q4, 64), F.Q4, 8, 64, 64)
    xs = torch.zeros(4 * 64 + 1, dtype=torch.int16, device="cuda:0")
    with pytest.raises(hip.QsfHipError):
        t4.prefill(xs[1:], 4, y)                # x not 16-byte aligned
    t4.free()


@pytest.mark.parametrize("m,n,k,bs", [(37, 100, 256, 64), (513, 129, 4096, 64), (64, 96, 768, 256)])
def test_packed_halves_equal_one_call(hip, m, n, k, bs):
    """prefill_pack once + the packed GEMM of two tensors that share x give
    the bits of one qsf_hip_prefill_4bit_dev call per tensor."""
    torch = torch_cuda()
    stream = torch.cuda.current_stream()
    pa, xb = case(7 + m, m, n, k, bs)
    pb, _ = case(8 + m, m, n, k, bs)
    dx = torch.from_numpy(xb.view(np.int16).copy()).to("cuda:0")
    ta, tb = hip.Tensor(pa, F.Q4, n, k, bs), hip.Tensor(pb, F.Q4, n, k, bs)
    try:
        packed = torch.empty(hip.prefill_pack_bytes(m, k, bs) + 256, dtype=torch.uint8, device="cuda:0")
        paddr = (packed.data_ptr() + 255) & ~255
        hip.prefill_pack(dx, m, k, bs, paddr, stream=stream)
        outs = []
        for t in (ta, tb):
            y1 = torch.full((m, n), float("nan"), device="cuda:0")
            y2 = torch.full((m, n), float("nan"), device="cuda:0")
            t.prefill(dx, m, y1, stream=stream)
            t.prefill_packed(paddr, m, y2, stream=stream)
            outs.append((y1, y2))
        torch.cuda.synchronize()
        for y1, y2 in outs:
            assert np.array_equal(y1.cpu().numpy().view(np.uint32), y2.cpu().numpy().view(np.uint32))
    finally:
        ta.free()
        tb.free()


def test_stream_read_floor_runs(hip):
    """The bare-read diagnostic launch completes over tensors of every kind
    (dense, outlier CSR, MXFP4) and stores nothing to its sink."""
    torch = torch_cuda()
    rng = np.random.default_rng(3)
    ts = [hip.Tensor(F.quantize_matrix(F.gaussian(rng, (300, 1000), 0.02), F.Q4, 64), F.Q4, 300, 1000, 64),
          hip.Tensor(F.quantize_matrix(F.heavy_tail_weights(rng, 64, 4096), F.Q2_OUTLIER, 64), F.Q2_OUTLIER,
                     64, 4096, 64),
          hip.Tensor(F.random_mxfp4(rng, 96, 2880), F.MXFP4, 96, 2880, 32)]
    try:
        sink = torch.zeros(1, dtype=torch.int32, device="cuda:0")
        hip.stream_read(ts, sink, stream=torch.cuda.current_stream())
        torch.cuda.synchronize()
        assert int(sink.cpu()[0]) == 0
    finally:
        for t in ts:
            t.free()


def test_mfma_peak_probe(hip):
    """The bf16 matrix-core probe the bench sets the prefill beside: one
    launch returns its FLOP (every CU's waves, 8 chains of iters
    v_mfma_f32_16x16x32_bf16 each), leaves the sink alone in practice, and
    refuses a bad count."""
    torch = torch_cuda()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.zeros(4, dtype=torch.int32, device="cuda:0")
    flop = hip.mfma_peak(16, sink, stream=torch.cuda.current_stream())
    torch.cuda.synchronize()
    assert flop == cus * 4 * 4 * 16 * 8 * 2 * 16 * 16 * 32
    assert int(sink.cpu()[0]) == 0
    with pytest.raises(hip.QsfHipError):
        hip.mfma_peak(0, sink)
