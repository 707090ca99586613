"""The C ABI: libqsf_hip loads and exports every function include/qsf_hip.h
declares (no GPU calls), and the table-slot layout matches QStream's
QSFKernelTable."""
from __future__ import annotations

import ctypes as C
import os
import re
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qsf_hip.h")
REF_INCLUDE = "/root/reference/include"


def declared_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(qsf_\w+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_entry_points():
    names = declared_functions()
    for must in ("qsf_matvec_4bit_hip", "qsf_matvec_outlier_2bit_hip", "qsf_kernels_init_hip",
                 "qsf_hip_matvec_dev", "qsf_hip_moe_forward_dev", "qsf_hip_unpack_dev"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from qstream_amd import qsf_hip
    lib = qsf_hip.load()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(qsf_hip.EXPORTS) <= set(declared_functions())


def test_oracle_library_loads():
    from oracle.oracle import Oracle
    o = Oracle()
    assert o.block_bytes(3, 64) == 36 and o.block_bytes(0, 64) == 20 and o.block_bytes(2, 128) == 52


def test_table_init_writes_six_slots():
    """qsf_kernels_init_hip fills slots 0..5 and leaves the rest alone."""
    from qstream_amd import qsf_hip
    lib = qsf_hip.load()
    table = (C.c_void_p * 18)(*([0xDEAD] * 18))
    mx = C.c_void_p(0)
    lib.qsf_kernels_init_hip(C.cast(table, C.c_void_p), None, C.byref(mx))
    want = [C.cast(getattr(lib, f"qsf_{s}_hip"), C.c_void_p).value for s in qsf_hip.MATVEC_SLOTS]
    assert list(table[:6]) == want
    assert all(v == 0xDEAD for v in table[6:])
    assert mx.value == C.cast(lib.qsf_matvec_mxfp4_hip, C.c_void_p).value


@pytest.mark.skipif(not os.path.isdir(REF_INCLUDE), reason="reference headers absent")
def test_slot_offsets_match_reference_table():
    """Compile against include/qsf/kernels.h: the six matvec slots are the
    first six pointers of QSFKernelTable (include/qsf/kernels.h:91-98)."""
    src = r'''
#include <stddef.h>
#include <stdio.h>
#include "qsf/kernels.h"
int main(void) {
    printf("%zu %zu %zu %zu %zu %zu %zu\n",
        offsetof(QSFKernelTable, matvec_2bit), offsetof(QSFKernelTable, matvec_3bit),
        offsetof(QSFKernelTable, matvec_4bit), offsetof(QSFKernelTable, matvec_4bit_sym),
        offsetof(QSFKernelTable, matvec_outlier_2bit), offsetof(QSFKernelTable, matvec_outlier_4bit),
        sizeof(void*));
    return 0;
}
'''
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "t.c")
        exe = os.path.join(d, "t")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-std=c11", f"-I{REF_INCLUDE}", c, "-o", exe], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split()
    offs = [int(v) for v in out]
    assert offs[:6] == [i * offs[6] for i in range(6)]


def test_missing_library_fails_loudly(tmp_path):
    from qstream_amd import qsf_hip
    with pytest.raises(qsf_hip.QsfHipError):
        qsf_hip.load.__wrapped__(str(tmp_path / "nope.so")) if hasattr(qsf_hip.load, "__wrapped__") \
            else _load_fresh(qsf_hip, str(tmp_path / "nope.so"))


def _load_fresh(mod, path):
    saved = mod._lib
    mod._lib = None
    try:
        return mod.load(path)
    finally:
        mod._lib = saved


DROPIN = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref",
                      "dropin_table")


@pytest.mark.skipif(not os.path.exists(DROPIN), reason="oracle/_ref not built (reference sources absent)")
def test_real_kernel_table_takeover():
    """oracle/dropin_table: the reference's qsf_kernels_init fills a real
    QSFKernelTable (src/kernels.c:7-65), qsf_kernels_init_hip takes over the
    six matvec members and the MXFP4 slot, and the other twelve members stay
    the CPU kernels (no GPU call)."""
    from qstream_amd import qsf_hip
    r = subprocess.run([DROPIN, qsf_hip.LIB_PATH, "--slots-only"], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 0 and r.stdout.strip().endswith("OK"), r.stdout + r.stderr
