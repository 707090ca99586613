"""GPT-OSS MXFP4 experts -> QSF MoE tensor records (quant type 11).

The reference converter loads GPT-OSS's packed expert tensors
(tools/convert_hf.py:1296-1308), dequantises them and quantises them again
to the file's block type.  Two things in that path are wrong, and this
writer fixes both:

* Scale.  The reference multiplies each code by the raw E8M0 byte
  (``scales.float()``, tools/convert_hf.py:1314-1317).  An E8M0 byte E
  encodes 2^(E-127), and 255 encodes NaN (OCP Microscaling Formats v1.0,
  section 5.4.1).  ``dequant_mxfp4`` uses that.
* gate/up split.  ``gate_up_proj`` holds the gate and up rows interleaved:
  GPT-OSS computes ``gate_up = x @ W + b`` and then takes ``gate_up[..., ::2]``
  as gate and ``gate_up[..., 1::2]`` as up (the published model code,
  transformers ``models/gpt_oss/modeling_gpt_oss.py``, ``GptOssExperts``).
  Blocks are stored [experts][output rows][blocks][16], so gate is the even
  output rows and up the odd ones.  The reference splits by halves
  (tools/convert_hf.py:1328-1336 and 1345-1352 for the bias), which pairs
  gate channel i with channel i + I instead of 2i+1.  ``split="halves"``
  reproduces that for comparison.

With ``quant=MXFP4`` (the default) the experts are not re-quantised: each
expert's rows are cut from the checkpoint's bytes and written as the QSF
MXFP4 payload, codes plane [rows][cols/32][16] then E8M0 plane
[rows][cols/32] (the layout ``qsf_matvec_mxfp4_hip`` reads).  Every byte of
the payload is a byte of the checkpoint, so nothing is lost.  Any other
``quant`` dequantises with the fixed scale and re-quantises with
``qsf_format.quantize_matrix``, as the reference converter does.

Tensor records follow the reference layer writer
(tools/convert_hf.py:1083-1211): weights as matrices, biases as FP16
vectors, router weights in the layer's dense type, the router bias as an
FP16 vector, expert tensors typed QSF_MOE_*(e) (include/qsf/types.h:145-162).
"""
from __future__ import annotations

from typing import Mapping

import numpy as np

from . import qsf_format as F

# OCP MX v1.0 E2M1 values by code (sign bit 3); the element order inside a
# byte (even element in the low nibble) is that of tools/convert_hf.py:1456-1495.
E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                 -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], np.float32)


def e8m0_scale(e) -> np.ndarray:
    """2^(E-127) for E8M0 bytes E, NaN for 255 (OCP MX v1.0)."""
    e = np.asarray(e, np.uint8)
    out = np.ldexp(np.float32(1.0), np.minimum(e.astype(np.int32), 254) - 127).astype(np.float32)
    return np.where(e == 255, np.float32(np.nan), out)


def dequant_mxfp4(blocks: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """[..., B, 16] uint8 codes and [..., B] E8M0 scales -> [..., B*32] fp32."""
    blocks = np.asarray(blocks, np.uint8)
    lo, hi = E2M1[blocks & 15], E2M1[blocks >> 4]
    vals = np.stack([lo, hi], axis=-1).reshape(*blocks.shape[:-1], 32)
    vals = vals * e8m0_scale(scales)[..., None]
    return vals.reshape(*blocks.shape[:-2], blocks.shape[-2] * 32).astype(np.float32)


def split_gate_up(a: np.ndarray, split: str = "interleave"):
    """Split a gate_up tensor along its output-row axis (axis 1 of an
    [experts][rows]... array, or the last axis of a [experts][rows] bias)."""
    axis = 1
    n = a.shape[axis]
    if n % 2:
        raise ValueError(f"gate_up has an odd number of rows ({n})")
    if split == "interleave":
        return np.take(a, np.arange(0, n, 2), axis), np.take(a, np.arange(1, n, 2), axis)
    if split == "halves":
        return np.take(a, np.arange(n // 2), axis), np.take(a, np.arange(n // 2, n), axis)
    raise ValueError(f"split must be 'interleave' or 'halves', not {split!r}")


def mxfp4_payload(blocks: np.ndarray, scales: np.ndarray) -> bytes:
    """QSF MXFP4 payload of one matrix: [rows][B][16] codes, [rows][B] scales."""
    blocks = np.ascontiguousarray(blocks, np.uint8)
    scales = np.ascontiguousarray(scales, np.uint8)
    if blocks.ndim != 3 or blocks.shape[2] != 16 or scales.shape != blocks.shape[:2]:
        raise ValueError(f"blocks {blocks.shape} / scales {scales.shape} are not [R][B][16] / [R][B]")
    return blocks.tobytes() + scales.tobytes()


def _fp16_bytes(v) -> bytes:
    return np.ascontiguousarray(np.asarray(v, np.float32).astype(np.float16)).tobytes()


def _vector(ttype: int, v) -> tuple:
    v = np.asarray(v, np.float32).reshape(-1)
    return (ttype, F.FP16, 1, v.size, _fp16_bytes(v))


def _expert_matrix(ttype, blocks, scales, quant, bs):
    rows, nblk = scales.shape
    if quant == F.MXFP4:
        return (ttype, F.MXFP4, rows, nblk * 32, mxfp4_payload(blocks, scales))
    w = dequant_mxfp4(blocks, scales)
    return (ttype, quant, rows, w.shape[1], F.quantize_matrix(w, quant, bs))


def moe_layer_records(t: Mapping[str, np.ndarray], layer: int, *, quant: int = F.MXFP4,
                      dense_quant: int = F.Q4, block_size: int = 64,
                      split: str = "interleave") -> list:
    """Tensor records of one GPT-OSS layer's MoE block.

    ``t`` maps checkpoint names to arrays: ``model.layers.{i}.mlp.experts.``
    ``gate_up_proj_blocks`` [E][2I][H/32][16], ``gate_up_proj_scales``
    [E][2I][H/32], ``down_proj_blocks`` [E][H][I/32][16],
    ``down_proj_scales`` [E][H][I/32], optional ``gate_up_proj_bias`` [E][2I]
    and ``down_proj_bias`` [E][H]; ``model.layers.{i}.mlp.router.weight``
    [E][H] and optional ``router.bias`` [E]."""
    p = f"model.layers.{layer}.mlp"
    gub, gus = t[f"{p}.experts.gate_up_proj_blocks"], t[f"{p}.experts.gate_up_proj_scales"]
    db, ds = t[f"{p}.experts.down_proj_blocks"], t[f"{p}.experts.down_proj_scales"]
    n_exp = gub.shape[0]
    if gus.shape != gub.shape[:3] or ds.shape != db.shape[:3] or db.shape[0] != n_exp:
        raise ValueError("expert blocks and scales disagree in shape")
    (gb, ub), (gs, us) = split_gate_up(gub, split), split_gate_up(gus, split)
    gu_bias = t.get(f"{p}.experts.gate_up_proj_bias")
    g_bias, u_bias = split_gate_up(np.asarray(gu_bias, np.float32), split) if gu_bias is not None \
        else (None, None)
    d_bias = t.get(f"{p}.experts.down_proj_bias")
    recs = []
    router = t.get(f"{p}.router.weight")
    if router is not None:
        router = np.asarray(router, np.float32)
        recs.append((F.T_MOE_ROUTER, dense_quant, router.shape[0], router.shape[1],
                     F.quantize_matrix(router, dense_quant, block_size)))
    if t.get(f"{p}.router.bias") is not None:
        recs.append(_vector(F.T_MOE_ROUTER_BIAS, t[f"{p}.router.bias"]))
    for e in range(n_exp):
        recs.append(_expert_matrix(F.t_moe(e, "gate"), gb[e], gs[e], quant, block_size))
        if g_bias is not None:
            recs.append(_vector(F.t_moe(e, "gate", True), g_bias[e]))
        recs.append(_expert_matrix(F.t_moe(e, "up"), ub[e], us[e], quant, block_size))
        if u_bias is not None:
            recs.append(_vector(F.t_moe(e, "up", True), u_bias[e]))
        recs.append(_expert_matrix(F.t_moe(e, "down"), db[e], ds[e], quant, block_size))
        if d_bias is not None:
            recs.append(_vector(F.t_moe(e, "down", True), np.asarray(d_bias, np.float32)[e]))
    return recs


def load_gpt_oss_layer(path: str, layer: int) -> dict:
    """The MoE tensors of one layer from a safetensors file, as numpy
    (bf16 tensors widened to fp32 exactly; codes and scales as uint8)."""
    from safetensors import safe_open
    p = f"model.layers.{layer}.mlp."
    out = {}
    with safe_open(path, framework="pt", device="cpu") as f:
        for k in f.keys():
            if not k.startswith(p):
                continue
            v = f.get_tensor(k)
            out[k] = v.float().numpy() if v.is_floating_point() else v.numpy()
    return out
