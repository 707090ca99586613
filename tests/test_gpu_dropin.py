"""The engine's own way into the library, on the GPU: oracle/dropin_table
(built from QStream's kernels.c and CPU kernels with this tree's
dropin_table.c) fills a real QSFKernelTable with qsf_kernels_init
(src/kernels.c:7-65), lets qsf_kernels_init_hip take over the matvec
members, and calls each slot through its struct member as engine.c does
(src/engine.c:141-152): 36 cases (6 types x 6 shapes) within relative L2
1e-5 of the reference's scalar kernels and of the CPU slots it replaced,
except the AVX2 4-bit symmetric slot, which reads codes as q - 8
(src/kernels_avx2.c:300-302) where the scalar kernel this library follows
reads them as two's complement (src/quant.c:158-177): its disagreement is
printed, not held to the bar."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

DROPIN = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref",
                      "dropin_table")


@pytest.mark.skipif(not os.path.exists(DROPIN), reason="oracle/_ref not built")
def test_kernel_table_slots_through_the_struct():
    from qstream_amd import qsf_hip
    print("dropin_table: every matvec slot through QSFKernelTable", flush=True)
    r = subprocess.run([DROPIN, qsf_hip.LIB_PATH], capture_output=True, text=True, timeout=100)
    print(r.stdout[-3000:], flush=True)
    assert r.returncode == 0 and r.stdout.strip().endswith("OK"), r.stdout + r.stderr
