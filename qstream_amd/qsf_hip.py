"""ctypes binding of libqsf_hip (include/qsf_hip.h).

Mirrors QStream's kernel-table interface (include/qsf/kernels.h:91-126):
``KernelTable().matvec_4bit(w, x, out, rows, cols, bs)`` has the argument
meaning of ``qsf_matvec_fn`` and, like it, returns nothing and overwrites
``out``.  The device entry points take torch CUDA tensors (or raw device
addresses) and a stream.

Loading fails loudly when the built library is missing: there is no CPU
fallback on this path.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libqsf_hip.so")

_vp, _i, _fp = C.c_void_p, C.c_int, C.POINTER(C.c_float)

MATVEC_SLOTS = ("matvec_2bit", "matvec_3bit", "matvec_4bit", "matvec_4bit_sym",
                "matvec_outlier_2bit", "matvec_outlier_4bit")
EXPORTS = (
    "qsf_hip_init", "qsf_hip_shutdown", "qsf_hip_last_error", "qsf_hip_last_error_detail",
    "qsf_matvec_2bit_hip", "qsf_matvec_3bit_hip", "qsf_matvec_4bit_hip",
    "qsf_matvec_4bit_sym_hip", "qsf_matvec_outlier_2bit_hip", "qsf_matvec_outlier_4bit_hip",
    "qsf_matvec_mxfp4_hip", "qsf_kernels_init_hip", "qsf_hip_slot_lookahead",
    "qsf_hip_tensor_upload", "qsf_hip_tensor_upload_pair", "qsf_hip_tensor_lookup", "qsf_hip_tensor_free",
    "qsf_hip_arena_forget", "qsf_hip_arena_forget_range", "qsf_hip_arena_bytes", "qsf_hip_tensor_payload_bytes",
    "qsf_hip_matvec_dev", "qsf_hip_matvec_group_dev", "qsf_hip_xprep_bytes",
    "qsf_hip_xprep_dev", "qsf_hip_matvec_group_prepared_dev",
    "qsf_hip_moe_create", "qsf_hip_moe_free", "qsf_hip_moe_forward_dev",
    "qsf_hip_unpack_dev", "qsf_hip_kernel_timing", "qsf_hip_kernel_timing_read", "qsf_hip_gemv_engine", "qsf_hip_moe_stages",
    "qsf_hip_prefill_4bit_dev", "qsf_hip_prefill_4bit_dev_noalloc", "qsf_hip_prefill_pack_bytes",
    "qsf_hip_prefill_pack_dev", "qsf_hip_prefill_4bit_packed_dev", "qsf_hip_stream_read_dev", "qsf_hip_mfma_peak_dev",
    "qsf_hip_rms_norm_dev", "qsf_hip_layer_norm_dev", "qsf_hip_rope_create", "qsf_hip_rope_free",
    "qsf_hip_rope_dev", "qsf_hip_kv_store_dev", "qsf_hip_attention_dev", "qsf_hip_act_mul_dev",
    "qsf_hip_gate_up_act_dev", "qsf_hip_residual_dev", "qsf_hip_embed_row_dev", "qsf_hip_embed_row_fp16_dev",
    "qsf_hip_residual_norm_dev", "qsf_hip_rope_kv_store_dev", "qsf_hip_rope_kv_attention_dev",
    "qsf_hip_residual_norm_matvec_group_dev", "qsf_hip_residual_norm_gate_up_act_dev",
    "qsf_hip_crc32", "qsf_hip_model_load", "qsf_hip_model_load_mem", "qsf_hip_model_free", "qsf_hip_model_get_info",
    "qsf_hip_model_tensor", "qsf_hip_model_vector", "qsf_hip_model_embedding",
    "qsf_hip_model_embedding_fp16", "qsf_hip_model_output_head", "qsf_hip_model_final_norm", "qsf_hip_model_moe",
)

_lib = None


class QsfHipError(RuntimeError):
    pass


def load(path: str = LIB_PATH) -> C.CDLL:
    """Load libqsf_hip.so (built by qstream_amd.build); raise if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise QsfHipError(f"{path} is not built: run `python -m qstream_amd.build`")
    # One HIP runtime per process: when torch is present its bundled
    # libamdhip64 (soname libamdhip64.so.7) must be loaded first so this
    # library's DT_NEEDED binds to it instead of pulling in a second runtime.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    L = C.CDLL(path)
    L.qsf_hip_init.argtypes = [_i]
    L.qsf_hip_init.restype = _i
    L.qsf_hip_last_error.restype = _i
    L.qsf_hip_last_error_detail.restype = C.c_char_p
    for s in MATVEC_SLOTS + ("matvec_mxfp4",):
        f = getattr(L, f"qsf_{s}_hip")
        f.argtypes = [_vp, _vp, _vp, _i, _i, _i]
        f.restype = None
    L.qsf_kernels_init_hip.argtypes = [_vp, _vp, C.POINTER(_vp)]
    L.qsf_hip_tensor_upload.argtypes = [_vp, _i, _i, _i, _i]
    L.qsf_hip_tensor_upload.restype = _vp
    L.qsf_hip_tensor_lookup.argtypes = [_vp]
    L.qsf_hip_tensor_lookup.restype = _vp
    L.qsf_hip_tensor_free.argtypes = [_vp]
    L.qsf_hip_arena_forget.argtypes = [_vp]
    L.qsf_hip_arena_forget_range.argtypes = [_vp, C.c_size_t]
    L.qsf_hip_slot_lookahead.argtypes = [_i]
    L.qsf_hip_slot_lookahead.restype = _i
    L.qsf_hip_arena_bytes.restype = C.c_size_t
    L.qsf_hip_tensor_payload_bytes.argtypes = [_vp]
    L.qsf_hip_tensor_payload_bytes.restype = C.c_size_t
    L.qsf_hip_matvec_dev.argtypes = [_vp, _vp, _vp, _vp]
    L.qsf_hip_matvec_dev.restype = _i
    L.qsf_hip_matvec_group_dev.argtypes = [C.POINTER(_vp), _i, _vp, C.POINTER(_vp), _vp]
    L.qsf_hip_matvec_group_dev.restype = _i
    L.qsf_hip_xprep_bytes.argtypes = [_i, _i, _i]
    L.qsf_hip_xprep_bytes.restype = C.c_size_t
    L.qsf_hip_xprep_dev.argtypes = [_i, _i, _i, _vp, _vp, _vp]
    L.qsf_hip_xprep_dev.restype = _i
    L.qsf_hip_matvec_group_prepared_dev.argtypes = [C.POINTER(_vp), _i, _vp, _vp, C.POINTER(_vp), _vp]
    L.qsf_hip_matvec_group_prepared_dev.restype = _i
    L.qsf_hip_moe_create.argtypes = [_i, _i, _i] + [C.POINTER(_vp)] * 6
    L.qsf_hip_moe_create.restype = _vp
    L.qsf_hip_moe_free.argtypes = [_vp]
    L.qsf_hip_moe_forward_dev.argtypes = [_vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp]
    L.qsf_hip_moe_forward_dev.restype = _i
    L.qsf_hip_unpack_dev.argtypes = [_i, _vp, _i, _i, _vp, _vp, _vp, _vp]
    L.qsf_hip_unpack_dev.restype = _i
    L.qsf_hip_prefill_4bit_dev.argtypes = [_vp, _vp, _i, _vp, _vp]
    L.qsf_hip_prefill_4bit_dev.restype = _i
    L.qsf_hip_prefill_4bit_dev_noalloc.argtypes = [_vp, _vp, _i, _vp, _vp]
    L.qsf_hip_prefill_4bit_dev_noalloc.restype = _i
    L.qsf_hip_prefill_pack_bytes.argtypes = [_i, _i, _i]
    L.qsf_hip_prefill_pack_bytes.restype = C.c_size_t
    L.qsf_hip_prefill_pack_dev.argtypes = [_vp, _i, _i, _i, _vp, _vp]
    L.qsf_hip_prefill_pack_dev.restype = _i
    L.qsf_hip_prefill_4bit_packed_dev.argtypes = [_vp, _vp, _i, _vp, _vp]
    L.qsf_hip_prefill_4bit_packed_dev.restype = _i
    L.qsf_hip_stream_read_dev.argtypes = [C.POINTER(_vp), _i, _vp, _vp]
    L.qsf_hip_stream_read_dev.restype = _i
    L.qsf_hip_mfma_peak_dev.argtypes = [_i, _vp, _vp]
    L.qsf_hip_mfma_peak_dev.restype = C.c_double
    _f = C.c_float
    L.qsf_hip_rms_norm_dev.argtypes = [_vp, _vp, _vp, _i, _f, _vp]
    L.qsf_hip_layer_norm_dev.argtypes = [_vp, _vp, _vp, _vp, _i, _f, _vp]
    L.qsf_hip_rope_create.argtypes = [_i, _f]
    L.qsf_hip_rope_create.restype = _vp
    L.qsf_hip_rope_free.argtypes = [_vp]
    L.qsf_hip_rope_dev.argtypes = [_vp, _vp, _vp, _i, _i, _i, _vp]
    L.qsf_hip_kv_store_dev.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp]
    L.qsf_hip_attention_dev.argtypes = [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _vp]
    L.qsf_hip_act_mul_dev.argtypes = [_vp, _vp, _i, _i, _vp]
    L.qsf_hip_gate_up_act_dev.argtypes = [_vp, _vp, _vp, _i, _vp]
    L.qsf_hip_tensor_upload_pair.argtypes = [_vp, _vp, _i, _i, _i, _i]
    L.qsf_hip_tensor_upload_pair.restype = _vp
    L.qsf_hip_residual_dev.argtypes = [_vp, _vp, _i, _vp, _vp]
    L.qsf_hip_embed_row_dev.argtypes = [_vp, _i, _vp, _vp]
    L.qsf_hip_embed_row_fp16_dev.argtypes = [_vp, _i, _i, _vp, _vp]
    L.qsf_hip_residual_norm_dev.argtypes = [_vp, _vp, _i, _vp, _vp, _vp, _f, _i, _vp, _vp]
    L.qsf_hip_residual_norm_matvec_group_dev.argtypes = [_vp, _i, _vp, _vp, _vp, _vp, _vp, _f, _vp, _vp]
    L.qsf_hip_residual_norm_gate_up_act_dev.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _f, _vp, _i, _vp]
    L.qsf_hip_rope_kv_store_dev.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, _i, _vp]
    L.qsf_hip_rope_kv_attention_dev.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, _i, _vp,
                                                _vp]
    for n in ("qsf_hip_rms_norm_dev", "qsf_hip_layer_norm_dev", "qsf_hip_rope_dev",
              "qsf_hip_kv_store_dev", "qsf_hip_attention_dev", "qsf_hip_act_mul_dev",
              "qsf_hip_gate_up_act_dev", "qsf_hip_residual_dev", "qsf_hip_embed_row_dev", "qsf_hip_embed_row_fp16_dev",
              "qsf_hip_residual_norm_dev", "qsf_hip_rope_kv_store_dev", "qsf_hip_rope_kv_attention_dev",
              "qsf_hip_residual_norm_matvec_group_dev", "qsf_hip_residual_norm_gate_up_act_dev"):
        getattr(L, n).restype = _i
    L.qsf_hip_crc32.argtypes = [_vp, C.c_size_t]
    L.qsf_hip_crc32.restype = C.c_uint32
    L.qsf_hip_model_load.argtypes = [C.c_char_p]
    L.qsf_hip_model_load.restype = _vp
    L.qsf_hip_model_load_mem.argtypes = [_vp, C.c_size_t]
    L.qsf_hip_model_load_mem.restype = _vp
    L.qsf_hip_model_free.argtypes = [_vp]
    L.qsf_hip_model_get_info.argtypes = [_vp, _vp]
    L.qsf_hip_model_get_info.restype = _i
    L.qsf_hip_model_tensor.argtypes = [_vp, _i, _i]
    L.qsf_hip_model_tensor.restype = _vp
    L.qsf_hip_model_vector.argtypes = [_vp, _i, _i, C.POINTER(_i)]
    L.qsf_hip_model_vector.restype = _vp
    for n in ("qsf_hip_model_embedding", "qsf_hip_model_embedding_fp16", "qsf_hip_model_output_head"):
        getattr(L, n).argtypes = [_vp]
        getattr(L, n).restype = _vp
    L.qsf_hip_model_final_norm.argtypes = [_vp, C.POINTER(_vp)]
    L.qsf_hip_model_final_norm.restype = _vp
    L.qsf_hip_model_moe.argtypes = [_vp, _i]
    L.qsf_hip_model_moe.restype = _vp
    L.qsf_hip_kernel_timing.argtypes = [_i]
    L.qsf_hip_kernel_timing.restype = _i
    L.qsf_hip_kernel_timing_read.argtypes = [C.POINTER(C.c_float), _i]
    L.qsf_hip_kernel_timing_read.restype = _i
    L.qsf_hip_gemv_engine.argtypes = [_i]
    L.qsf_hip_gemv_engine.restype = _i
    L.qsf_hip_moe_stages.argtypes = [_i]
    L.qsf_hip_moe_stages.restype = _i
    _lib = L
    return L


def gemv_engine(engine: int = -1) -> int:
    """Decode GEMV engine for tensors uploaded from now on: 1 (default) the
    int8 matrix-core kernel for 3-bit tensors, 2 for every format it covers,
    0 the dot-product kernels for all; < 0 queries.  Returns the previous
    setting."""
    return int(load().qsf_hip_gemv_engine(engine))


def moe_stages(mask: int = -1) -> int:
    """Stages Moe.forward launches from now on (measurement aid): bit 0
    routing, bit 1 gate/up, bit 2 down + combine; 7 by default; < 0
    queries.  Returns the previous mask."""
    return int(load().qsf_hip_moe_stages(mask))


def kernel_timing(enable: bool) -> None:
    """Record an event pair at each decode GEMV kernel's own start and end."""
    _check(load().qsf_hip_kernel_timing(1 if enable else 0), "qsf_hip_kernel_timing")


def kernel_timing_read(max_n: int = 4096):
    """Durations (us) of the launches recorded since timing was enabled."""
    import numpy as np
    buf = (C.c_float * max_n)()
    n = load().qsf_hip_kernel_timing_read(buf, max_n)
    if n < 0:
        _check(n, "qsf_hip_kernel_timing_read")
    return np.frombuffer(buf, dtype=np.float32, count=n).copy()


def last_error() -> tuple[int, str]:
    L = load()
    d = L.qsf_hip_last_error_detail()
    return L.qsf_hip_last_error(), (d.decode() if d else "")


def _check(rc: int, what: str) -> None:
    if rc != 0:
        code, detail = last_error()
        raise QsfHipError(f"{what} failed ({rc}): {detail}")


def _addr(t) -> int:
    """Device address of a torch tensor, or an int address."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(s) -> int | None:
    if s is None:
        return None
    if isinstance(s, int):
        return s
    return s.cuda_stream


def init(device: int = 0) -> None:
    _check(load().qsf_hip_init(device), "qsf_hip_init")


def arena_forget(payload) -> bool:
    """Drop the arena entry (and volatile mark) of a host payload buffer;
    False when the buffer was not registered."""
    a = payload if isinstance(payload, np.ndarray) else np.frombuffer(payload, np.uint8)
    return load().qsf_hip_arena_forget(a.ctypes.data) == 0


def arena_forget_range(buf) -> int:
    """Forget every registered pointer inside a host buffer; returns how many."""
    a = buf if isinstance(buf, np.ndarray) else np.frombuffer(buf, np.uint8)
    return load().qsf_hip_arena_forget_range(a.ctypes.data, a.nbytes)


def arena_forget_all() -> int:
    """Forget every registered host pointer (the table slots upload their
    payloads afresh); returns how many."""
    return load().qsf_hip_arena_forget_range(None, C.c_size_t(-1).value)


def slot_lookahead(n: int = -1) -> int:
    """Successors a table-slot call may run in its own launch (0 = off);
    n < 0 only queries.  Returns the previous setting."""
    return load().qsf_hip_slot_lookahead(int(n))


class KernelTable:
    """The six matvec slots of QSFKernelTable backed by libqsf_hip.

    Each slot takes (weights_q: bytes|np.ndarray, input: float32[cols],
    output: float32[rows], rows, cols, block_size) like qsf_matvec_fn.
    """

    def __init__(self):
        self._L = load()
        for s in MATVEC_SLOTS + ("matvec_mxfp4",):
            setattr(self, s, self._slot(getattr(self._L, f"qsf_{s}_hip")))
        self._keep = []

    def _slot(self, fn):
        def call(w, x, out, rows, cols, bs):
            wa = np.frombuffer(w, np.uint8) if isinstance(w, (bytes, bytearray)) else w
            self._keep.append(wa)   # the library keys uploaded payloads by address
            if not (out.dtype == np.float32 and out.flags.c_contiguous):
                raise TypeError("output must be a contiguous float32 array")
            xa = np.ascontiguousarray(x, np.float32)
            fn(wa.ctypes.data, xa.ctypes.data, out.ctypes.data, rows, cols, bs)
        return call


class Tensor:
    """A weight payload resident in HBM (device weight arena)."""

    def __init__(self, payload, qt: int, rows: int, cols: int, bs: int):
        self._host = np.frombuffer(payload, np.uint8) if isinstance(payload, (bytes, bytearray)) \
            else np.ascontiguousarray(payload)
        self.qt, self.rows, self.cols, self.bs = qt, rows, cols, bs
        L = load()
        self.handle = L.qsf_hip_tensor_upload(self._host.ctypes.data, qt, rows, cols, bs)
        if not self.handle:
            _check(-1, "qsf_hip_tensor_upload")
        self.payload_bytes = L.qsf_hip_tensor_payload_bytes(self.handle)

    def prefill(self, x_bf16, m: int, y, stream=None) -> None:
        """y[m][rows] = W . float(x_bf16[m][cols]) on MFMA (4-bit tensors)."""
        _check(load().qsf_hip_prefill_4bit_dev(self.handle, _addr(x_bf16), m, _addr(y),
                                               _stream(stream)), "qsf_hip_prefill_4bit_dev")

    def prefill_noalloc(self, x_bf16, m: int, y, stream=None) -> None:
        """The same through the allocation-free entry point (static per-GPU
        scratch; safe to capture into a graph without a first eager call)."""
        _check(load().qsf_hip_prefill_4bit_dev_noalloc(self.handle, _addr(x_bf16), m, _addr(y),
                                                       _stream(stream)),
               "qsf_hip_prefill_4bit_dev_noalloc")

    def prefill_packed(self, packed, m: int, y, stream=None) -> None:
        """The GEMM half of prefill over activations prefill_pack wrote."""
        _check(load().qsf_hip_prefill_4bit_packed_dev(self.handle, _addr(packed), m, _addr(y),
                                                      _stream(stream)), "qsf_hip_prefill_4bit_packed_dev")

    def matvec(self, x, y, stream=None) -> None:
        _check(load().qsf_hip_matvec_dev(self.handle, _addr(x), _addr(y), _stream(stream)),
               "qsf_hip_matvec_dev")

    def free(self) -> None:
        if self.handle:
            load().qsf_hip_tensor_free(self.handle)
            self.handle = None


class TensorPair(Tensor):
    """Gate and up payloads of one FFN as one interleaved HBM tensor
    (2 * rows rows) for gate_up_act."""

    def __init__(self, gate, up, qt: int, rows: int, cols: int, bs: int):
        as_u8 = lambda p: np.frombuffer(p, np.uint8) if isinstance(p, (bytes, bytearray)) \
            else np.ascontiguousarray(p)
        g, u = as_u8(gate), as_u8(up)
        self.qt, self.rows, self.cols, self.bs = qt, rows, cols, bs
        L = load()
        self.handle = L.qsf_hip_tensor_upload_pair(g.ctypes.data, u.ctypes.data, qt, rows, cols, bs)
        if not self.handle:
            _check(-1, "qsf_hip_tensor_upload_pair")
        self.payload_bytes = L.qsf_hip_tensor_payload_bytes(self.handle)

    def residual_norm_gate_up_act(self, res, res_out, x, w, eps, out, activation, bad=None,
                                  stream=None) -> None:
        """res_out = res + x (NaN check into `bad`), then out = act(gate n) * (up n) for
        n = rms_norm(res_out) * w, in one launch."""
        _check(load().qsf_hip_residual_norm_gate_up_act_dev(self.handle, _addr(res), _addr(res_out),
                                                            _addr(x), _addr(bad), _addr(w), eps,
                                                            _addr(out), activation, _stream(stream)),
               "qsf_hip_residual_norm_gate_up_act_dev")

    def gate_up_act(self, x, out, activation, stream=None) -> None:
        """out[i] = act(gate_i . x) * (up_i . x) in one launch."""
        _check(load().qsf_hip_gate_up_act_dev(self.handle, _addr(x), _addr(out), activation,
                                              _stream(stream)), "qsf_hip_gate_up_act_dev")


def prefill_pack_bytes(m: int, cols: int, bs: int) -> int:
    return int(load().qsf_hip_prefill_pack_bytes(m, cols, bs))


def prefill_pack(x_bf16, m: int, cols: int, bs: int, packed, stream=None) -> None:
    """x bf16 [m][cols] into `packed` (prefill_pack_bytes bytes, 16-byte
    aligned), shared by every 4-bit tensor of these cols and block size."""
    _check(load().qsf_hip_prefill_pack_dev(_addr(x_bf16), m, cols, bs, _addr(packed), _stream(stream)),
           "qsf_hip_prefill_pack_dev")


def mfma_peak(iters, sink, stream=None) -> float:
    """One launch of independent bf16 MFMA chains on every CU; returns its FLOP."""
    flop = load().qsf_hip_mfma_peak_dev(iters, _addr(sink), _stream(stream))
    if flop < 0:
        _check(-1, "qsf_hip_mfma_peak_dev")
    return float(flop)


def stream_read(tensors, sink, stream=None) -> None:
    """One launch streaming the tensors' device bytes once (the bare-read floor)."""
    n = len(tensors)
    th = (_vp * n)(*[t.handle for t in tensors])
    _check(load().qsf_hip_stream_read_dev(th, n, _addr(sink), _stream(stream)), "qsf_hip_stream_read_dev")


def matvec_group(tensors, x, ys, stream=None) -> None:
    n = len(tensors)
    th = (_vp * n)(*[t.handle for t in tensors])
    yh = (_vp * n)(*[_addr(y) for y in ys])
    _check(load().qsf_hip_matvec_group_dev(th, n, _addr(x), yh, _stream(stream)),
           "qsf_hip_matvec_group_dev")


def residual_norm_matvec_group(tensors, res, res_out, x, w, eps, ys, bad=None, stream=None) -> None:
    """res_out = res + x (NaN check into `bad`), then ys[i] = tensors[i] . (rms_norm(res_out) * w),
    in one launch."""
    n = len(tensors)
    th = (_vp * n)(*[t.handle for t in tensors])
    yh = (_vp * n)(*[_addr(y) for y in ys])
    _check(load().qsf_hip_residual_norm_matvec_group_dev(th, n, _addr(res), _addr(res_out), _addr(x),
                                                         _addr(bad), _addr(w), eps, yh, _stream(stream)),
           "qsf_hip_residual_norm_matvec_group_dev")


def xprep_bytes(qt: int, bs: int, cols: int) -> int:
    return load().qsf_hip_xprep_bytes(qt, bs, cols)


def xprep(qt: int, bs: int, cols: int, x, xq, stream=None) -> None:
    _check(load().qsf_hip_xprep_dev(qt, bs, cols, _addr(x), _addr(xq), _stream(stream)),
           "qsf_hip_xprep_dev")


def matvec_group_prepared(tensors, x, xq, ys, stream=None) -> None:
    n = len(tensors)
    th = (_vp * n)(*[t.handle for t in tensors])
    yh = (_vp * n)(*[_addr(y) for y in ys])
    _check(load().qsf_hip_matvec_group_prepared_dev(th, n, _addr(x), _addr(xq), yh, _stream(stream)),
           "qsf_hip_matvec_group_prepared_dev")


def unpack(qt: int, d_blocks, nblocks: int, bs: int, codes=None, meta=None, deq=None,
           stream=None) -> None:
    _check(load().qsf_hip_unpack_dev(qt, _addr(d_blocks), nblocks, bs, _addr(codes),
                                     _addr(meta), _addr(deq), _stream(stream)),
           "qsf_hip_unpack_dev")


class Moe:
    """Device expert table for the MXFP4 MoE FFN (src/engine.c:951-1107)."""

    def __init__(self, gate, up, down, hidden: int, eid: int,
                 gate_bias=None, up_bias=None, down_bias=None):
        n = len(gate)
        self.n_exp, self.hidden, self.eid = n, hidden, eid
        self._keep = [gate, up, down]
        arr = lambda ts: (_vp * n)(*[t.handle for t in ts])

        def biases(bs):
            if bs is None:
                return None
            hs = [None if b is None else np.ascontiguousarray(b, np.uint16) for b in bs]
            self._keep.append(hs)
            return (_vp * n)(*[None if b is None else b.ctypes.data for b in hs])
        L = load()
        self.handle = L.qsf_hip_moe_create(n, hidden, eid, arr(gate), arr(up), arr(down),
                                           biases(gate_bias), biases(up_bias), biases(down_bias))
        if not self.handle:
            _check(-1, "qsf_hip_moe_create")

    def forward(self, k, norm_topk, act, ntok, x, logits, out, stream=None) -> None:
        _check(load().qsf_hip_moe_forward_dev(self.handle, k, norm_topk, act, ntok, _addr(x),
                                              _addr(logits), _addr(out), _stream(stream)),
               "qsf_hip_moe_forward_dev")

    def free(self) -> None:
        if self.handle:
            load().qsf_hip_moe_free(self.handle)
            self.handle = None


# ---- device-resident decode glue (src/engine.c:709-1187) --------------------
def rms_norm(x, out, w, eps, stream=None) -> None:
    _check(load().qsf_hip_rms_norm_dev(_addr(x), _addr(out), _addr(w), x.numel(), eps,
                                       _stream(stream)), "qsf_hip_rms_norm_dev")


def layer_norm(x, out, w, b, eps, stream=None) -> None:
    _check(load().qsf_hip_layer_norm_dev(_addr(x), _addr(out), _addr(w), _addr(b), x.numel(), eps,
                                         _stream(stream)), "qsf_hip_layer_norm_dev")


class Rope:
    """RoPE frequency table on the device (qsf_hip_rope_create)."""

    def __init__(self, head_dim: int, theta: float):
        self.head_dim = head_dim
        self.handle = load().qsf_hip_rope_create(head_dim, theta)
        if not self.handle:
            _check(-1, "qsf_hip_rope_create")

    def apply(self, q, k, n_heads, n_kv, position, stream=None) -> None:
        _check(load().qsf_hip_rope_dev(self.handle, _addr(q), _addr(k), n_heads, n_kv, position,
                                       _stream(stream)), "qsf_hip_rope_dev")

    def apply_and_store(self, q, k, v, n_heads, n_kv, position, kc, vc, ks, vs, max_seq,
                        stream=None) -> None:
        """RoPE of q and k, then the int8 KV store of k and v, in one launch."""
        _check(load().qsf_hip_rope_kv_store_dev(self.handle, _addr(q), _addr(k), _addr(v), n_heads,
                                                n_kv, position, _addr(kc), _addr(vc), _addr(ks),
                                                _addr(vs), max_seq, _stream(stream)),
               "qsf_hip_rope_kv_store_dev")

    def apply_store_attend(self, q, k, v, n_heads, n_kv, position, kc, vc, ks, vs, max_seq, out,
                           stream=None) -> None:
        """apply_and_store then attention(), with the RoPE, the KV store and
        the attention's chunk pass in one launch for head_dim 64/128/256;
        q and k are not read afterwards (rotated in place or not)."""
        _check(load().qsf_hip_rope_kv_attention_dev(self.handle, _addr(q), _addr(k), _addr(v), n_heads, n_kv,
                                                    position, _addr(kc), _addr(vc), _addr(ks), _addr(vs),
                                                    max_seq, _addr(out), _stream(stream)),
               "qsf_hip_rope_kv_attention_dev")

    def free(self) -> None:
        if self.handle:
            load().qsf_hip_rope_free(self.handle)
            self.handle = None


def kv_store(kc, vc, ks, vs, max_seq, n_kv, head_dim, position, k, v, stream=None) -> None:
    _check(load().qsf_hip_kv_store_dev(_addr(kc), _addr(vc), _addr(ks), _addr(vs), max_seq, n_kv,
                                       head_dim, position, _addr(k), _addr(v), _stream(stream)),
           "qsf_hip_kv_store_dev")


def attention(q, kc, vc, ks, vs, max_seq, n_heads, n_kv, head_dim, position, out,
              stream=None) -> None:
    _check(load().qsf_hip_attention_dev(_addr(q), _addr(kc), _addr(vc), _addr(ks), _addr(vs),
                                        max_seq, n_heads, n_kv, head_dim, position, _addr(out),
                                        _stream(stream)), "qsf_hip_attention_dev")


def act_mul(gate, up, activation, stream=None) -> None:
    _check(load().qsf_hip_act_mul_dev(_addr(gate), _addr(up), gate.numel(), activation,
                                      _stream(stream)), "qsf_hip_act_mul_dev")


def residual(res, x, bad=None, stream=None) -> None:
    _check(load().qsf_hip_residual_dev(_addr(res), _addr(x), res.numel(), _addr(bad),
                                       _stream(stream)), "qsf_hip_residual_dev")


def residual_norm(res, x, w, eps, out, bad=None, b=None, layer_norm=False, stream=None) -> None:
    """res += x (with the NaN check into `bad`), then out = norm(res), in one launch."""
    _check(load().qsf_hip_residual_norm_dev(_addr(res), _addr(x), res.numel(), _addr(bad), _addr(w),
                                            _addr(b), eps, int(layer_norm), _addr(out),
                                            _stream(stream)), "qsf_hip_residual_norm_dev")


def embed_row(table: "Tensor", token: int, out, stream=None) -> None:
    _check(load().qsf_hip_embed_row_dev(table.handle, token, _addr(out), _stream(stream)),
           "qsf_hip_embed_row_dev")


def embed_row_fp16(d_table, hd: int, token: int, out, stream=None) -> None:
    _check(load().qsf_hip_embed_row_fp16_dev(_addr(d_table), hd, token, _addr(out),
                                             _stream(stream)), "qsf_hip_embed_row_fp16_dev")


# ---- QSF model file -> device arena ------------------------------------------
class ModelInfo(C.Structure):
    """qsf_hip_model_info (include/qsf_hip.h)."""
    _fields_ = [(n, C.c_uint32) for n in (
        "num_layers", "hidden_dim", "num_heads", "num_kv_heads", "vocab_size", "max_seq_len",
        "intermediate_dim", "head_dim", "block_size", "quant_type", "activation", "norm_type",
        "pos_enc_type", "ffn_type", "attn_type", "has_bias", "weight_tied", "num_experts",
        "num_active_experts", "expert_intermediate_dim", "moe_norm_topk")] + [
        ("rope_theta", C.c_float), ("norm_epsilon", C.c_float), ("num_tensors", C.c_uint32),
        ("has_embedding", C.c_uint32), ("crc_mismatches", C.c_uint32),
        ("size_mismatch", C.c_uint32), ("moe_layers", C.c_uint32), ("device_bytes", C.c_size_t)]


def crc32(data: bytes) -> int:
    buf = np.frombuffer(data, np.uint8)
    return load().qsf_hip_crc32(buf.ctypes.data, len(buf))


class _Ref:
    """A tensor the model owns (no free)."""

    def __init__(self, handle):
        self.handle = handle

    def matvec(self, x, y, stream=None) -> None:
        _check(load().qsf_hip_matvec_dev(self.handle, _addr(x), _addr(y), _stream(stream)),
               "qsf_hip_matvec_dev")


class Model:
    """A QSF file loaded into the device arena (qsf_hip_model_load)."""

    def __init__(self, path: str):
        L = load()
        self.handle = L.qsf_hip_model_load(path.encode())
        if not self.handle:
            code, detail = last_error()
            raise QsfHipError(f"qsf_hip_model_load failed ({code}): {detail}")
        self.info = ModelInfo()
        _check(L.qsf_hip_model_get_info(self.handle, C.byref(self.info)), "qsf_hip_model_get_info")

    def tensor(self, layer: int, tensor_type: int):
        h = load().qsf_hip_model_tensor(self.handle, layer, tensor_type)
        return _Ref(h) if h else None

    def vector(self, layer: int, tensor_type: int):
        n = C.c_int(0)
        p = load().qsf_hip_model_vector(self.handle, layer, tensor_type, C.byref(n))
        return (p, n.value) if p else (None, 0)

    def embedding(self):
        h = load().qsf_hip_model_embedding(self.handle)
        return _Ref(h) if h else None

    def embedding_fp16(self) -> int | None:
        """Device address of an FP16 embedding table [vocab][hidden], or None."""
        return load().qsf_hip_model_embedding_fp16(self.handle) or None

    def output_head(self):
        h = load().qsf_hip_model_output_head(self.handle)
        return _Ref(h) if h else None

    def moe(self, layer: int):
        """The layer's device MXFP4 expert table (forward like Moe), or None."""
        h = load().qsf_hip_model_moe(self.handle, layer)
        if not h:
            return None
        m = Moe.__new__(Moe)
        m.handle, m._keep = h, [self]
        m.free = lambda: None          # owned by the model
        return m

    def final_norm(self):
        b = _vp()
        w = load().qsf_hip_model_final_norm(self.handle, C.byref(b))
        return w, b.value

    def free(self) -> None:
        if self.handle:
            load().qsf_hip_model_free(self.handle)
            self.handle = None

