"""Device block orders (no GPU calls): row-plane order, as the library's own
qk_plane_offset addresses it, is a permutation of each row's bytes that keeps
every block's meta dword and every 64-code part's code bytes whole and in
order, so a 16-byte load of a plane reads whole aligned runs."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

BITS = {0: 2, 1: 3, 2: 4, 3: 4}       # QK_FMT_2, _3, _4, _4SYM


@pytest.fixture(scope="module")
def off():
    from qstream_amd import qsf_hip
    f = qsf_hip.load().qk_plane_offset
    f.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]
    f.restype = C.c_size_t
    return f


@pytest.mark.parametrize("fmt", [0, 1, 2])
@pytest.mark.parametrize("bs", [32, 64, 128, 256])
@pytest.mark.parametrize("nb", [1, 3, 64])
def test_plane_order_is_a_permutation_of_each_row(off, fmt, bs, nb):
    bb = 4 + bs * BITS[fmt] // 8
    pos = np.array([[off(b, j, nb, bb, bs) for j in range(bb)] for b in range(nb)], np.int64)
    assert sorted(pos.ravel().tolist()) == list(range(nb * bb))
    if bs <= 64:
        # plane i holds bytes [16 i, 16 i + 16) of block b at 16 b, contiguous
        for i in range(bb // 16):
            assert np.array_equal(pos[:, 16 * i:16 * i + 16],
                                  i * nb * 16 + 16 * np.arange(nb)[:, None] + np.arange(16))
        tb = bb % 16
        tail = (bb // 16) * nb * 16 + tb * np.arange(nb)[:, None] + np.arange(tb)
        assert np.array_equal(pos[:, bb - tb:], tail)
    else:
        # the meta dwords first, then each 64-code part's code bytes in order
        assert np.array_equal(pos[:, :4], 4 * np.arange(nb)[:, None] + np.arange(4))
        P, cwb = bs // 64, (bb - 4) // (bs // 64)
        for p in range(P):
            part = pos[:, 4 + p * cwb:4 + (p + 1) * cwb]
            u = np.arange(nb) * P + p
            assert np.array_equal(part[:, :16], 4 * nb + 16 * u[:, None] + np.arange(16))
            assert (np.diff(part, axis=1)[:, :15] == 1).all()


def test_plane_order_moves_bytes_on_disk_order_would_not(off):
    """A 2-bit block of 64 codes (20 bytes): block 1's meta is not at byte 20,
    its tail dword is in the tail plane after the 16-byte plane."""
    nb, bb = 4, 20
    assert off(1, 0, nb, bb, 64) == 16
    assert off(1, 16, nb, bb, 64) == nb * 16 + 4
