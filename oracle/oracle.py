"""ctypes bindings of the CPU parity checker (test infrastructure only).

``Oracle`` wraps this build's C restatement (liboracle.so); ``RefLib`` wraps
QStream's own quant.c/kernels_scalar.c/kernels_avx2.c compiled from the
reference tree into oracle/_ref (present only where it was built).
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module; the product path never does.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_STRICT_SO = os.path.join(HERE, "_ref", "libqsf_ref_strict.so")
REF_AVX2_SO = os.path.join(HERE, "_ref", "libqsf_ref_avx2.so")

_vp, _fp, _i = C.c_void_p, C.POINTER(C.c_float), C.c_int


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _buf(b):
    """bytes / uint8 array -> (keepalive array, void*)."""
    a = np.frombuffer(b, dtype=np.uint8) if isinstance(b, (bytes, bytearray)) else np.ascontiguousarray(b)
    return a, _ptr(a)


class Oracle:
    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = self.lib = C.CDLL(path)
        L.orc_fp16_to_fp32.restype = C.c_float
        L.orc_fp16_to_fp32.argtypes = [C.c_uint16]
        L.orc_fp16_to_fp32_array.argtypes = [_vp, _vp, _i]
        L.orc_block_bytes.restype = C.c_size_t
        L.orc_block_bytes.argtypes = [_i, _i]
        L.orc_unpack_codes.argtypes = [_i, _vp, _i, _vp]
        L.orc_dequant_block.argtypes = [_i, _vp, _vp, _i]
        L.orc_unpack_codes_many.argtypes = [_i, _vp, _i, _i, _vp]
        L.orc_matvec.argtypes = [_i, _vp, _vp, _vp, _i, _i, _i]
        L.orc_payload_bytes.restype = C.c_size_t
        L.orc_payload_bytes.argtypes = [_i, _vp, _i, _i, _i]
        L.orc_e2m1_to_fp32.restype = C.c_float
        L.orc_e2m1_to_fp32.argtypes = [C.c_uint8]
        L.orc_e8m0_to_fp32.restype = C.c_float
        L.orc_e8m0_to_fp32.argtypes = [C.c_uint8]
        L.orc_softmax.argtypes = [_vp, _vp, _i]
        L.orc_act.argtypes = [_i, _vp, _i]
        L.orc_topk.argtypes = [_vp, _i, _i, _i, _vp, _vp]
        L.orc_moe_token.argtypes = [_vp, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp]
        L.orc_prefill_4bit.argtypes = [_vp, _vp, _vp, _i, _i, _i, _i]
        L.orc_rms_norm.argtypes = [_vp, _vp, _vp, _i, C.c_float]
        L.orc_layer_norm.argtypes = [_vp, _vp, _vp, _vp, _i, C.c_float]
        L.orc_vec_add.argtypes = [_vp, _vp, _vp, _i]
        L.orc_vec_mul.argtypes = [_vp, _vp, _vp, _i]
        L.orc_rope.argtypes = [_vp, _vp, _i, _i, C.c_float, _i, _i]
        L.orc_kv_store.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp]
        L.orc_attention.argtypes = [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]
        L.orc_residual_check.argtypes = [_vp, _vp, _i]
        L.orc_residual_check.restype = _i
        L.orc_embed_row.argtypes = [_i, _vp, _i, _i, _i, _vp]

    def fp16_to_fp32_bits(self, h: np.ndarray) -> np.ndarray:
        # bulk C call: a ctypes float return would quiet signalling NaNs
        h = np.ascontiguousarray(h, np.uint16)
        out = np.empty(len(h), np.float32)
        self.lib.orc_fp16_to_fp32_array(_ptr(h), _ptr(out), len(h))
        return out.view(np.uint32)

    def block_bytes(self, qt: int, bs: int) -> int:
        return self.lib.orc_block_bytes(qt, bs)

    def unpack_codes(self, qt: int, block, count: int) -> np.ndarray:
        keep, p = _buf(block)
        out = np.zeros(count, np.int8)
        self.lib.orc_unpack_codes(qt, p, count, _ptr(out))
        return out

    def dequant_block(self, qt: int, block, count: int) -> np.ndarray:
        keep, p = _buf(block)
        out = np.zeros(count, np.float32)
        self.lib.orc_dequant_block(qt, p, _ptr(out), count)
        return out

    def unpack_codes_many(self, qt: int, blocks, nblocks: int, bs: int) -> np.ndarray:
        keep, p = _buf(blocks)
        out = np.zeros(nblocks * bs, np.int8)
        self.lib.orc_unpack_codes_many(qt, p, nblocks, bs, _ptr(out))
        return out.reshape(nblocks, bs)

    def matvec(self, qt: int, payload, x: np.ndarray, rows: int, cols: int, bs: int) -> np.ndarray:
        keep, p = _buf(payload)
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(max(rows, 0), np.float32)
        self.lib.orc_matvec(qt, p, _ptr(x), _ptr(y), rows, cols, bs)
        return y

    def payload_bytes(self, qt, payload, rows, cols, bs) -> int:
        keep, p = _buf(payload)
        return self.lib.orc_payload_bytes(qt, p, rows, cols, bs)

    def softmax(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros_like(x)
        self.lib.orc_softmax(_ptr(x), _ptr(out), len(x))
        return out

    def act(self, act: int, x):
        x = np.array(x, np.float32, copy=True)
        self.lib.orc_act(act, _ptr(x), len(x))
        return x

    def topk(self, probs, k: int, norm: int):
        probs = np.ascontiguousarray(probs, np.float32)
        idx = np.zeros(k, np.int32)
        w = np.zeros(k, np.float32)
        self.lib.orc_topk(_ptr(probs), len(probs), k, norm, _ptr(idx), _ptr(w))
        return idx, w

    def moe_token(self, experts, k, norm, act, hidden, eid, x, logits):
        """experts: list of dicts with gate/up/down payload bytes and optional
        fp16 bias arrays (gate_bias, up_bias, down_bias)."""
        class Ex(C.Structure):
            _fields_ = [(n, C.c_void_p) for n in
                        ("gate", "gate_bias", "up", "up_bias", "down", "down_bias")]
        keep = []
        arr = (Ex * len(experts))()
        for i, e in enumerate(experts):
            for n in ("gate", "gate_bias", "up", "up_bias", "down", "down_bias"):
                v = e.get(n)
                if v is None:
                    setattr(arr[i], n, None)
                    continue
                a, p = _buf(v if not isinstance(v, np.ndarray) else np.ascontiguousarray(v))
                keep.append(a)
                setattr(arr[i], n, p.value)
        x = np.ascontiguousarray(x, np.float32)
        logits = np.ascontiguousarray(logits, np.float32)
        out = np.zeros(hidden, np.float32)
        self.lib.orc_moe_token(C.cast(arr, C.c_void_p), len(experts), k, norm, act,
                               hidden, eid, _ptr(x), _ptr(logits), _ptr(out))
        return out

    def prefill_4bit(self, payload, x_bf16: np.ndarray, m, n, k, bs) -> np.ndarray:
        keep, p = _buf(payload)
        xb = np.ascontiguousarray(x_bf16, np.uint16)
        y = np.zeros((m, n), np.float32)
        self.lib.orc_prefill_4bit(p, _ptr(xb), _ptr(y), m, n, k, bs)
        return y


    # ---- decode glue (src/engine.c, src/kernels_scalar.c) ----------------
    def rms_norm(self, x, w, eps):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        out = np.empty_like(x)
        self.lib.orc_rms_norm(_ptr(x), _ptr(out), _ptr(w), len(x), eps)
        return out

    def layer_norm(self, x, w, b, eps):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        bb = None if b is None else np.ascontiguousarray(b, np.float32)
        out = np.empty_like(x)
        self.lib.orc_layer_norm(_ptr(x), _ptr(out), _ptr(w), None if bb is None else _ptr(bb),
                                len(x), eps)
        return out

    def rope(self, q, k, head_dim, position, theta, n_heads, n_kv):
        q = np.array(q, np.float32, copy=True)
        k = np.array(k, np.float32, copy=True)
        self.lib.orc_rope(_ptr(q), _ptr(k), head_dim, position, theta, n_heads, n_kv)
        return q, k

    def kv_store(self, kc, vc, ks, vs, max_seq, n_kv, head_dim, position, k, v):
        """Writes row `position` of the layer's int8 caches in place."""
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        self.lib.orc_kv_store(_ptr(kc), _ptr(vc), _ptr(ks), _ptr(vs), max_seq, n_kv, head_dim,
                              position, _ptr(k), _ptr(v))

    def attention(self, q, kc, vc, ks, vs, max_seq, n_heads, n_kv, head_dim, position):
        q = np.ascontiguousarray(q, np.float32)
        out = np.zeros(n_heads * head_dim, np.float32)
        self.lib.orc_attention(_ptr(q), _ptr(kc), _ptr(vc), _ptr(ks), _ptr(vs), max_seq, n_heads,
                               n_kv, head_dim, position, _ptr(out))
        return out

    def residual_check(self, res, x):
        res = np.array(res, np.float32, copy=True)
        x = np.ascontiguousarray(x, np.float32)
        bad = self.lib.orc_residual_check(_ptr(res), _ptr(x), len(res))
        return res, bad

    def embed_row(self, qt, table, bs, hd, token):
        keep, p = _buf(table)
        out = np.zeros(hd, np.float32)
        self.lib.orc_embed_row(qt, p, bs, hd, token, _ptr(out))
        return out

    def vec_add(self, a, b):
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        out = np.empty_like(a)
        self.lib.orc_vec_add(_ptr(a), _ptr(b), _ptr(out), len(a))
        return out

    def vec_mul(self, a, b):
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        out = np.empty_like(a)
        self.lib.orc_vec_mul(_ptr(a), _ptr(b), _ptr(out), len(a))
        return out


_MATVEC_SYMS = ("qsf_matvec_2bit_scalar", "qsf_matvec_3bit_scalar",
                "qsf_matvec_4bit_scalar", "qsf_matvec_4bit_sym_scalar")
_AVX2_SYMS = ("qsf_matvec_2bit_avx2", "qsf_matvec_4bit_avx2",
              "qsf_matvec_4bit_sym_avx2", "qsf_matvec_outlier_2bit_avx2",
              "qsf_matvec_outlier_4bit_avx2")


class RefLib:
    """QStream's own hot-path translation units (compiled into oracle/_ref)."""

    def __init__(self, path: str):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.lib = C.CDLL(path)
        self.path = path
        L.qsf_fp16_to_fp32.restype = C.c_float
        L.qsf_fp16_to_fp32.argtypes = [C.c_uint16]
        L.qsf_fp16_to_fp32_array.argtypes = [_vp, _vp, _i]
        L.qsf_quant_block_size.restype = C.c_size_t
        L.qsf_quant_block_size.argtypes = [_i, _i]
        for n in ("qsf_dequant_block_2bit", "qsf_dequant_block_3bit",
                  "qsf_dequant_block_4bit", "qsf_dequant_block_4bit_sym"):
            getattr(L, n).argtypes = [_vp, _vp, _i]
        for n in _MATVEC_SYMS:
            getattr(L, n).argtypes = [_vp, _vp, _vp, _i, _i, _i]
        for n in ("qsf_matvec_outlier_2bit", "qsf_matvec_outlier_4bit"):
            getattr(L, n).argtypes = [_vp, C.c_size_t, _vp, _vp, _i, _i, _i]
        self.has_avx2 = hasattr(L, "qsf_matvec_4bit_avx2")
        if self.has_avx2:
            for n in _AVX2_SYMS:
                getattr(L, n).argtypes = [_vp, _vp, _vp, _i, _i, _i]
        # the elementwise kernels of src/kernels_scalar.c:112-214
        L.qsf_rms_norm_scalar.argtypes = [_vp, _vp, _vp, _vp, _i, C.c_float]
        L.qsf_layer_norm_scalar.argtypes = [_vp, _vp, _vp, _vp, _i, C.c_float]
        L.qsf_softmax_scalar.argtypes = [_vp, _vp, _i]
        for n in ("qsf_silu_scalar", "qsf_gelu_scalar", "qsf_relu_scalar"):
            getattr(L, n).argtypes = [_vp, _i]
        for n in ("qsf_vec_add_scalar_impl", "qsf_vec_mul_scalar_impl"):
            getattr(L, n).argtypes = [_vp, _vp, _vp, _i]
        L.qsf_quant_block_2bit.argtypes = [_vp, _vp, _i]
        L.qsf_quant_block_3bit.argtypes = [_vp, _vp, _i]
        L.qsf_quant_block_4bit.argtypes = [_vp, _vp, _i]

    def fp16_table(self) -> np.ndarray:
        # qsf_fp16_to_fp32_array (src/quant.c:61-65) writes the bits directly
        h = np.arange(65536, dtype=np.uint16)
        out = np.empty(65536, np.float32)
        self.lib.qsf_fp16_to_fp32_array(_ptr(h), _ptr(out), 65536)
        return out.view(np.uint32)

    def dequant_block(self, qt: int, block, count: int) -> np.ndarray:
        name = {0: "2bit", 1: "2bit", 2: "3bit", 3: "4bit", 4: "4bit_sym"}[qt]
        keep, p = _buf(block)
        out = np.zeros(count, np.float32)
        getattr(self.lib, f"qsf_dequant_block_{name}")(p, _ptr(out), count)
        return out

    def matvec(self, qt: int, payload, x, rows, cols, bs, isa: str = "scalar") -> np.ndarray:
        keep, p = _buf(payload)
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(max(rows, 0), np.float32)
        if qt in (9, 10):
            base = "2bit" if qt == 9 else "4bit"
            if isa == "avx2":
                getattr(self.lib, f"qsf_matvec_outlier_{base}_avx2")(p, _ptr(x), _ptr(y), rows, cols, bs)
            else:
                getattr(self.lib, f"qsf_matvec_outlier_{base}")(p, 0, _ptr(x), _ptr(y), rows, cols, bs)
            return y
        name = {0: "2bit", 1: "2bit", 2: "3bit", 4: "4bit_sym"}.get(qt, "4bit")
        if isa == "avx2" and name != "3bit":
            fn = getattr(self.lib, f"qsf_matvec_{name}_avx2")
        else:
            fn = getattr(self.lib, f"qsf_matvec_{name}_scalar")
        fn(p, _ptr(x), _ptr(y), rows, cols, bs)
        return y


def ref_strict() -> RefLib | None:
    return RefLib(REF_STRICT_SO) if os.path.exists(REF_STRICT_SO) else None


def ref_avx2() -> RefLib | None:
    return RefLib(REF_AVX2_SO) if os.path.exists(REF_AVX2_SO) else None


REF_CONTAINER_SO = os.path.join(HERE, "_ref", "libqsf_ref_container.so")


class _RefSummary(C.Structure):
    _fields_ = [("rc", C.c_int32), ("head_dim", C.c_uint32), ("num_kv_heads", C.c_uint32)] + [
        (n, C.c_int32) for n in ("is_gated_ffn", "uses_rope", "uses_alibi", "has_bias_attn_qkv",
                                 "has_bias_attn_o", "has_bias_ffn", "has_bias_norm", "weight_tied")] + [
        ("file_size", C.c_uint64), ("header", C.c_uint8 * 256)]


class RefContainer:
    """QStream's own QSF reader (src/format.c, src/file_access.c, src/error.c
    compiled into oracle/_ref behind oracle/ref_container.c)."""

    def __init__(self, path: str = REF_CONTAINER_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.lib = C.CDLL(path)
        L.ref_container_load.argtypes = [C.c_char_p, C.POINTER(_RefSummary), _vp, C.c_uint32, _vp]
        L.ref_container_load.restype = _i
        L.ref_container_error.restype = C.c_char_p
        L.ref_layout_count.restype = _i
        L.ref_layout_name.argtypes = [_i]
        L.ref_layout_name.restype = C.c_char_p
        L.ref_layout_value.argtypes = [_i]
        L.ref_layout_value.restype = C.c_long
        self.layout = {L.ref_layout_name(i).decode(): L.ref_layout_value(i) for i in range(L.ref_layout_count())}

    def load(self, path: str, max_layers: int = 256) -> dict:
        """qsf_model_load (+ qsf_decompress_layer of every layer): the QSFError,
        the header bytes and derived fields as the reference holds them, the
        layer-index entries and each layer's data offset in the file."""
        s = _RefSummary()
        li = np.zeros(max_layers * self.layout["QSFLayerIndex"], np.uint8)
        offs = np.full(max_layers, -2, np.int64)
        rc = self.lib.ref_container_load(path.encode(), C.byref(s), _ptr(li), max_layers, _ptr(offs))
        out = {k: getattr(s, k) for k, _ in _RefSummary._fields_ if k != "header"}
        out.update(rc=rc, error=self.lib.ref_container_error().decode(errors="replace"),
                   header=bytes(s.header), layer_index=li.tobytes(), layer_data_off=offs)
        return out


def ref_container() -> RefContainer | None:
    return RefContainer() if os.path.exists(REF_CONTAINER_SO) else None


REF_GLUE_SO = os.path.join(HERE, "_ref", "libqsf_ref_glue.so")


class RefGlue:
    """QStream's own static engine helpers apply_rope (src/engine.c:205-234)
    and kv_cache_store (src/engine.c:240-293), compiled from engine.c into
    oracle/_ref behind oracle/ref_glue.c.  Loaded with lazy binding: the rest
    of engine.c's dependencies are never called, so never bound."""

    def __init__(self, path: str = REF_GLUE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.lib = C.CDLL(path, mode=os.RTLD_LAZY | os.RTLD_LOCAL)
        L.ref_glue_apply_rope.argtypes = [_vp, _vp, _i, _i, C.c_float, _i, _i]
        L.ref_glue_apply_rope.restype = None
        L.ref_glue_kv_store.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp]
        L.ref_glue_kv_store.restype = None

    def rope(self, q, k, head_dim, position, theta, n_heads, n_kv):
        q = np.array(q, np.float32, copy=True)
        k = np.array(k, np.float32, copy=True)
        self.lib.ref_glue_apply_rope(_ptr(q), _ptr(k), head_dim, position, theta, n_heads, n_kv)
        return q, k

    def kv_store(self, kc, vc, ks, vs, max_seq, n_kv, head_dim, position, k, v):
        """Writes row `position` of the layer's int8 caches in place."""
        assert n_kv <= 64
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        self.lib.ref_glue_kv_store(_ptr(kc), _ptr(vc), _ptr(ks), _ptr(vs), max_seq, n_kv, head_dim, position,
                                   _ptr(k), _ptr(v))


def ref_glue() -> RefGlue | None:
    return RefGlue() if os.path.exists(REF_GLUE_SO) else None
