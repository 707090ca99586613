"""Write the golden fixtures of tests/golden/ from QStream's own C code.

Runs here, where oracle/_ref holds quant.c + kernels_scalar.c (+ AVX2)
compiled from the reference tree (`make -C oracle`).  The fixtures are data
only -- inputs and the reference's outputs -- so tests can pin the oracle and
the GPU path where the reference tree is absent.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import ctypes as C
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle.oracle import ref_avx2, ref_strict  # noqa: E402
from qstream_amd import qsf_format as F        # noqa: E402

OUT = os.path.join(HERE, "qsf_ref_vectors.npz")


def ramp_case(ref, qt):
    """tests/test_core.c:597-677: 4x64 ramp quantised by the reference's own
    C block quantiser, then its scalar matvec."""
    rows, cols, bs = 4, 64, 64
    w = (np.arange(rows * cols, dtype=np.float32) / 256.0 - 0.5).reshape(rows, cols)
    x = np.arange(cols, dtype=np.float32) / 64.0 - 0.5
    bb = ref.lib.qsf_quant_block_size(qt, bs)
    packed = np.zeros(rows * bb, np.uint8)
    quant = ref.lib.qsf_quant_block_4bit if qt == F.Q4 else ref.lib.qsf_quant_block_2bit
    for r in range(rows):
        row = np.ascontiguousarray(w[r])
        quant(row.ctypes.data, packed[r * bb:].ctypes.data, bs)
    y = ref.matvec(qt, packed, x, rows, cols, bs)
    return packed, x, y


def main() -> None:
    ref = ref_strict()
    if ref is None:
        raise SystemExit("oracle/_ref not built: run `make -C oracle` where the reference tree exists")
    avx = ref_avx2()
    rng = np.random.default_rng(20261201)
    out: dict[str, np.ndarray] = {}

    # fp16 -> fp32 over all 65536 inputs (src/quant.c:11-39): digest + samples
    table = ref.fp16_table()
    out["fp16_table_sha256"] = np.frombuffer(hashlib.sha256(table.tobytes()).digest(), np.uint8)
    out["fp16_sample_in"] = np.arange(0, 65536, 97, dtype=np.uint16)
    out["fp16_sample_out"] = table[::97].copy()

    # block dequantisation (src/quant.c:95-177)
    for qt in (F.Q2, F.Q3, F.Q4, F.Q4SYM):
        for bs in (32, 64, 128, 256):
            bb = F.block_bytes(qt, bs)
            raw = rng.integers(0, 256, size=(6, bb), dtype=np.uint8)
            raw[:, 0:2] = (rng.standard_normal(6).astype(np.float32) * np.float32(0.05)).astype(np.float16).view(np.uint8).reshape(-1, 2)
            raw[:, 2:4] = rng.standard_normal(6).astype(np.float16).view(np.uint8).reshape(-1, 2)
            deq = np.stack([ref.dequant_block(qt, raw[i], bs) for i in range(6)])
            out[f"deq_q{qt}_bs{bs}_in"] = raw
            out[f"deq_q{qt}_bs{bs}_out"] = deq

    # matvecs: scalar (strict) outputs are the pinned values; AVX2 outputs
    # (reference release flags) are kept for information
    cases = []
    for qt in (F.Q2, F.Q3, F.Q4, F.Q4SYM, F.Q2_OUTLIER, F.Q4_OUTLIER):
        for bs in (32, 64, 128, 256):
            for rows, cols in ((8, 256), (5, 200), (3, bs // 2 + 1)):
                w = F.gaussian(rng, (rows, cols), 0.02)
                if qt in (F.Q2_OUTLIER, F.Q4_OUTLIER):
                    w = F.heavy_tail_weights(rng, rows, cols)
                x = F.gaussian(rng, cols)
                payload = np.frombuffer(F.quantize_matrix(w, qt, bs, 0.02), np.uint8)
                y = ref.matvec(qt, payload, x, rows, cols, bs)
                name = f"mv_q{qt}_bs{bs}_{rows}x{cols}"
                out[name + "_w"] = payload
                out[name + "_x"] = x
                out[name + "_y"] = y
                out[name + "_meta"] = np.array([qt, rows, cols, bs], np.int32)
                if avx is not None and qt != F.Q3:
                    out[name + "_yavx2"] = avx.matvec(qt, payload, x, rows, cols, bs, isa="avx2")
                cases.append(name)
    out["mv_cases"] = np.array(cases)

    for qt in (F.Q4, F.Q2):
        packed, x, y = ramp_case(ref, qt)
        out[f"ramp_q{qt}_w"] = packed
        out[f"ramp_q{qt}_x"] = x
        out[f"ramp_q{qt}_y"] = y

    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {os.path.getsize(OUT)} bytes, {len(cases)} matvec cases")


if __name__ == "__main__":
    main()
