"""Shared helpers of the GPU parity tests (imported by tests only)."""
from __future__ import annotations

import numpy as np

REL_L2 = 1e-5   # north_star bar: max relative L2 error vs the scalar reference


def rel_l2(y: np.ndarray, ref: np.ndarray) -> float:
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    num = np.linalg.norm(y - ref)
    if den == 0.0:
        return 0.0 if num == 0.0 else float("inf")
    return float(num / den)


def torch_cuda():
    import torch
    assert torch.cuda.is_available(), "GPU tests need cuda:0"
    return torch


def dev(a: np.ndarray):
    torch = torch_cuda()
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def host(t) -> np.ndarray:
    torch = torch_cuda()
    torch.cuda.synchronize()
    return t.cpu().numpy()


def device_floats(ptr: int, n: int) -> np.ndarray:
    """Copy n fp32 values from a raw device address (memory a library
    object owns) to the host with hipMemcpy of the HIP runtime this process
    already loaded (torch's)."""
    import ctypes as C
    torch_cuda().cuda.synchronize()
    path = next(line.split()[-1] for line in open("/proc/self/maps") if "libamdhip64" in line)
    rt = C.CDLL(path)
    rt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    out = np.empty(n, np.float32)
    assert rt.hipMemcpy(out.ctypes.data, ptr, 4 * n, 2) == 0       # 2 = device to host
    return out



# Decode GEMV engines a parity module runs under (the setting applies to the
# tensors uploaded while it holds): 0 the dot-product kernels for every
# format, 2 the int8 matrix-core kernel wherever it covers the shape.  The
# default, 1, is the matrix-core kernel for the 3-bit formats and the
# dot-product kernels for the rest: the two together cover it.
ENGINES = [0, 2]


def engine_hip(request):
    """Body of a module-scoped `hip` fixture parametrized over ENGINES.  The
    table slots' registered payloads are dropped on entry and exit, so that
    no slot serves a tensor uploaded under another engine."""
    from qstream_amd import qsf_hip
    qsf_hip.init(0)
    qsf_hip.arena_forget_all()
    old = qsf_hip.gemv_engine(request.param)
    yield qsf_hip
    qsf_hip.arena_forget_all()
    qsf_hip.gemv_engine(old)
