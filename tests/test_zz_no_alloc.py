"""Allocation-free prefill (qsf_hip_prefill_4bit_dev_noalloc) against the
workspace entry point it mirrors (qsf_hip_prefill_4bit_dev), through the C
ABI: the same kernels, so the outputs are bit-identical, and both meet the
1e-5 bar against the scalar oracle."""
import numpy as np
import pytest

from qstream_amd import qsf_format as F
from gpu_util import REL_L2, rel_l2, torch_cuda

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    from qstream_amd import qsf_hip
    qsf_hip.init(0)
    return qsf_hip


def bf16_rne(a32):
    b = np.ascontiguousarray(a32, np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def setup(hip, seed, m, n, k, bs):
    torch = torch_cuda()
    rng = np.random.default_rng(seed)
    payload = F.quantize_matrix(F.gaussian(rng, (n, k), 0.02), F.Q4, bs)
    xb = bf16_rne(rng.standard_normal((m, k)).astype(np.float32))
    t = hip.Tensor(payload, F.Q4, n, k, bs)
    dx = torch.from_numpy(xb.view(np.int16).copy()).to("cuda:0")
    return payload, xb, t, dx


def test_noalloc_matches_workspace_entry_two_calls(hip, oracle):
    """Two calls in a row, the second with fewer tokens and columns: each
    equals the workspace entry point's output and the oracle's to 1e-5."""
    torch = torch_cuda()
    stream = torch.cuda.current_stream()
    for seed, (m, n, k, bs) in enumerate([(200, 300, 1000, 64), (37, 100, 256, 128)]):
        payload, xb, t, dx = setup(hip, seed, m, n, k, bs)
        y_ws = torch.full((m, n), float("nan"), device="cuda:0")
        y_na = torch.full((m, n), float("nan"), device="cuda:0")
        t.prefill(dx, m, y_ws, stream=stream)
        t.prefill_noalloc(dx, m, y_na, stream=stream)
        torch.cuda.synchronize()
        a, b = y_ws.cpu().numpy(), y_na.cpu().numpy()
        ref = oracle.prefill_4bit(payload, xb, m, n, k, bs)
        err = rel_l2(b, ref)
        print(f"call {seed}: {m}x{n}x{k} bs{bs}: noalloc rel_l2 vs oracle {err:.3e}")
        assert np.array_equal(a, b)
        assert err <= REL_L2, err
        t.free()


def test_noalloc_graph_capture_without_warmup(hip, oracle):
    """Captured into a graph with no eager call first; each replay, with
    eager work and a synchronisation between, matches the eager result."""
    torch = torch_cuda()
    m, n, k, bs = 64, 224, 512, 64
    payload, xb, t, dx = setup(hip, 7, m, n, k, bs)
    ref = oracle.prefill_4bit(payload, xb, m, n, k, bs)
    y = torch.full((m, n), float("nan"), device="cuda:0")
    stream = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        t.prefill_noalloc(dx, m, y, stream=stream)
    torch.cuda.synchronize()
    y_eager = torch.full((m, n), float("nan"), device="cuda:0")
    t.prefill(dx, m, y_eager, stream=torch.cuda.current_stream())
    torch.cuda.synchronize()
    want = y_eager.cpu().numpy()
    assert rel_l2(want, ref) <= REL_L2
    for rep in range(3):
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        assert np.array_equal(got, want), f"replay {rep}"
    del g
    t.free()


def test_noalloc_rejects_more_than_its_scratch(hip):
    """4096 tokens x 4096 columns need about 38 MB of scratch: refused on
    the host, before any launch."""
    torch = torch_cuda()
    rng = np.random.default_rng(3)
    n, k, bs = 16, 4096, 64
    t = hip.Tensor(F.quantize_matrix(F.gaussian(rng, (n, k), 0.02), F.Q4, bs), F.Q4, n, k, bs)
    x = torch.zeros(64, dtype=torch.int16, device="cuda:0")
    y = torch.zeros(16, device="cuda:0")
    with pytest.raises(hip.QsfHipError, match="scratch"):
        t.prefill_noalloc(x, 4096, y)
    t.free()
