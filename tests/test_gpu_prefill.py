"""Batched prefill (config 4) on MFMA: Y[m] = W float(bf16 x[m]).

Two references:
* exact-weights: fp64 products of the same bf16 weights the kernel builds
  (w = fp32(s*q + z), rounded to bf16 with round-to-nearest-even) and bf16 x.
  The kernel only adds fp32 accumulation error: rel-L2 <= 1e-5.
* the scalar oracle (M token-by-token src/kernels_scalar.c:64-85 matvecs on
  float(bf16(x)), fp32 weights): the difference is the bf16 rounding of the
  weights that the prefill design prescribes.  bf16 keeps 8 significant bits,
  so each weight moves by at most 2^-8 of itself (about 1.6e-3 rms for
  uniformly spread rounding errors); the bound is that worst case, 2^-8.
"""
import numpy as np
import pytest

from qstream_amd import qsf_format as F
from gpu_util import rel_l2, torch_cuda

pytestmark = pytest.mark.gpu

REL_EXACT = 1e-5
REL_BF16 = 2.0 ** -8


@pytest.fixture(scope="module")
def hip():
    from qstream_amd import qsf_hip
    qsf_hip.init(0)
    return qsf_hip


def bf16_rne(a32: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even (finite inputs)."""
    b = np.ascontiguousarray(a32, np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f64(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def dequant_bf16(oracle, payload, n, k, bs) -> np.ndarray:
    """The kernel's weights: bf16(fp32(s*q + z)) as fp64 [n][k]."""
    nb = (k + bs - 1) // bs
    bb = 4 + bs // 2
    raw = np.frombuffer(payload, np.uint8)[:n * nb * bb]
    q = oracle.unpack_codes_many(F.Q4, raw.tobytes(), n * nb, bs).astype(np.float32)
    meta = raw.reshape(n * nb, bb)[:, :4].copy().view(np.uint16)
    s = oracle.fp16_to_fp32_bits(meta[:, 0]).view(np.float32)[:, None]
    z = oracle.fp16_to_fp32_bits(meta[:, 1]).view(np.float32)[:, None]
    w32 = (s * q.reshape(n * nb, bs)) + z            # s*q exact; one rounding in +
    w = bf16_to_f64(bf16_rne(w32.astype(np.float32))).reshape(n, nb * bs)
    return w[:, :k]


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


SHAPES = [(1, 64, 64, 64), (37, 100, 256, 64), (128, 64, 512, 64), (200, 300, 1000, 64),
          (130, 70, 512, 128), (64, 96, 768, 256), (513, 129, 4096, 64)]


@pytest.mark.parametrize("m,n,k,bs", SHAPES)
def test_prefill_exact_weights(hip, oracle, m, n, k, bs):
    payload, xb = case(m * 7 + n + k, m, n, k, bs)
    got = run(hip, payload, xb, m, n, k, bs)
    w = dequant_bf16(oracle, payload, n, k, bs)
    ref = bf16_to_f64(xb) @ w.T
    err = rel_l2(got, ref)
    print(f"prefill {m}x{n}x{k} bs{bs}: rel_l2 vs exact-weight fp64 = {err:.3e}")
    assert err <= REL_EXACT, err


@pytest.mark.parametrize("m,n,k,bs", SHAPES[:5])
def test_prefill_vs_scalar_oracle(hip, oracle, m, n, k, bs):
    payload, xb = case(m * 7 + n + k, m, n, k, bs)
    got = run(hip, payload, xb, m, n, k, bs)
    ref = oracle.prefill_4bit(payload, xb, m, n, k, bs)
    err = rel_l2(got, ref)
    print(f"prefill {m}x{n}x{k} bs{bs}: rel_l2 vs scalar oracle = {err:.3e}")
    assert err <= REL_BF16, err


def test_prefill_config4_rows(hip, oracle):
    """Benchmark config 4 (M=512, K=4096, N=14336, block 64): all outputs
    against the exact-weight fp64 reference."""
    m, n, k, bs = 512, 14336, 4096, 64
    payload, xb = case(4, m, n, k, bs)
    got = run(hip, payload, xb, m, n, k, bs)
    w = dequant_bf16(oracle, payload, n, k, bs)
    ref = bf16_to_f64(xb) @ w.T
    err = rel_l2(got, ref)
    print(f"prefill config 4: rel_l2 = {err:.3e}")
    assert err <= REL_EXACT, err


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
