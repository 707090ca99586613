"""The loader's parse path under AddressSanitizer and
UndefinedBehaviorSanitizer (tests/asan/Makefile): qsf_loader.c built with
both sanitizers, its device calls replaced by host reads of every byte the
real upload reads (tests/asan/host_double.c), fed seeded byte mutations of
QSF files of several shapes (tests/asan/mutate_loader.c).  Half of the
mutations land on the files' structure fields.  Every mutant must be
loaded or rejected with no sanitizer report; the sweep stops at the
first one."""
from __future__ import annotations

import os
import shutil
import struct
import subprocess

import pytest

from qstream_amd import qsf_format as F
from tests import container_models as CM

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "asan")
EXE = os.path.join(HERE, "_build", "mutate_loader")
ITERS = 4000


def structure_offsets(kw, offs, raw) -> list[int]:
    """Byte offsets of the fields a QSF reader parses (include/qsf/types.h:
    185-312): header fields, layer-index entries, each tensor record's
    header and outlier count, the embedding and final section headers."""
    hot = list(range(0, 184, 4)) + [48, 49, 50, 51, 140, 141, 142, 143, 172, 173, 174, 175, 176, 177]
    li = offs["layer_index"]
    for i in range(len(kw["layers"])):
        hot += [li + 48 * i + d for d in (0, 8, 12, 16, 17, 18, 20, 24, 28, 32, 36)]
    for i, recs in enumerate(kw["layers"]):
        p = offs["layer_offsets"][i]
        for ttype, qt, rows, cols, payload in recs:
            hot += [p + d for d in (0, 2, 3, 4, 8, 12, 16, 20)]
            if qt in (F.Q2_OUTLIER, F.Q4_OUTLIER) or (qt == 0xFF and kw["quant_type"] in (9, 10)):
                hot.append(p + 24)
            p += 24 + len(payload)
    if offs["embedding"]:
        hot += [offs["embedding"] + d for d in range(0, 36, 4)]
    if offs["final"]:
        hot += [offs["final"] + d for d in range(0, 16, 4)]
    return sorted(set(h for h in hot if h < len(raw)))


@pytest.fixture(scope="module")
def exe():
    if not shutil.which("gcc") or not shutil.which("make"):
        pytest.skip("gcc/make absent")
    r = subprocess.run(["make", "-s", "-C", HERE], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    return EXE


@pytest.mark.parametrize("name", ["dense", "dense_tied", "outlier_tied", "moe"])
def test_mutated_files_never_read_out_of_bounds(exe, tmp_path, name):
    kw = CM.all_models()[name]
    path = tmp_path / f"{name}.qsf"
    offs = F.write_qsf(str(path), **kw)
    raw = path.read_bytes()
    hot = tmp_path / "hot.txt"
    hot.write_text("\n".join(map(str, structure_offsets(kw, offs, raw))))
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=23",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1:exitcode=24")
    seed = str(sum(struct.unpack("<I", name.encode()[:4].ljust(4, b"\0"))))
    r = subprocess.run([exe, str(path), str(ITERS), seed, str(hot)], capture_output=True, text=True,
                       timeout=600, env=env)
    report = "\n".join(l for l in r.stderr.splitlines() if "CRC mismatch" not in l and "size mismatch" not in l)
    assert r.returncode == 0, report[-4000:]
    assert f"{ITERS} mutants" in r.stdout, r.stdout
