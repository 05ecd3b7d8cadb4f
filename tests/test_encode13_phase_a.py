"""Phase A of the n = 2^13 i16 encode on the matrix cores
(volta-zk_amd/csrc/enc13_mfma.hpp): the byte split of the inputs, the balanced
base-256 digits of the DFT matrix, the bias vector and the fold of the eight
position sums, built for the host from the same header (libgl64_check.so) and
checked against Python big integers.  The lane-by-lane emulation follows the
instruction's operand layout (lane l holds A[l & 15][16 (l >> 4) + j] and
B[16 (l >> 4) + j][l & 15]; register r of D holds C[4 (l >> 4) + r][l & 15]),
which a GPU probe of v_mfma_i32_16x16x64_i8 confirmed.  CPU only."""
import ctypes
import pathlib
import random

import numpy as np
import pytest

P = 0xFFFF_FFFF_0000_0001
BAL_MAX = 0x7F7F7F7F7F7F7F7F
LIB = pathlib.Path(__file__).resolve().parent.parent / "volta-zk_amd" / "libgl64_check.so"


@pytest.fixture(scope="module")
def glc():
    if not LIB.exists():
        pytest.fail("libgl64_check.so missing: run volta-zk_amd/build.py (or __graft_entry__.build())")
    L = ctypes.CDLL(str(LIB))
    L.glc_balanced_digit.restype, L.glc_balanced_digit.argtypes = ctypes.c_int, [ctypes.c_uint64, ctypes.c_int]
    L.glc_bias_digit.restype, L.glc_bias_digit.argtypes = ctypes.c_int, [ctypes.c_int]
    L.glc_recombine.restype, L.glc_recombine.argtypes = ctypes.c_uint64, [ctypes.POINTER(ctypes.c_int)]
    L.glc_enc13_phase_a.restype = None
    L.glc_enc13_phase_a.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    return L


def test_balanced_digits_represent_every_element(glc):
    rnd = random.Random(3)
    edge = [0, 1, 127, 128, 255, 256, BAL_MAX, BAL_MAX + 1, 1 << 63, (1 << 63) - (1 << 32) + 1, P - 1, P - 2,
            0x8080808080808080, 0xFFFFFFFF, 0x100000000]
    for c in edge + [rnd.randrange(P) for _ in range(3000)]:
        d = [glc.glc_balanced_digit(c, pos) for pos in range(8)]
        assert all(-128 <= x <= 127 for x in d), (hex(c), d)
        assert sum(x << (8 * pos) for pos, x in enumerate(d)) % P == c


def test_bias_vector_is_a_multiple_of_p(glc):
    b = [glc.glc_bias_digit(pos) for pos in range(8)]
    assert all((1 << 20) <= x < (1 << 20) + 256 for x in b)
    assert sum(x << (8 * pos) for pos, x in enumerate(b)) % P == 0


def test_recombine_folds_eight_position_sums(glc):
    rnd = random.Random(5)
    top = (1 << 21) + (1 << 9) - 1
    cases = [[0] * 8, [top] * 8, [top, 0] * 4, [0, top] * 4, [1 << 20] * 8]
    cases += [[rnd.randrange(top + 1) for _ in range(8)] for _ in range(3000)]
    for a in cases:
        r = glc.glc_recombine((ctypes.c_int * 8)(*a))
        assert r % P == sum(x << (8 * pos) for pos, x in enumerate(a)) % P


def _half_table():
    w = pow(7, (P - 1) >> 13, P)
    tw = [1] * 4096
    for e in range(1, 4096):
        tw[e] = tw[e - 1] * w % P
    return w, np.array(tw, dtype=np.uint64)


@pytest.mark.parametrize("cols,kind", [(2048, "uniform"), (2048, "extremes"), (2047, "top band"), (1000, "uniform"),
                                       (64, "uniform"), (1, "extremes")])
def test_phase_a_emulation_matches_big_ints(glc, cols, kind):
    w, tw = _half_table()
    g = np.random.Generator(np.random.PCG64(cols))
    if kind == "uniform":
        x = g.integers(-(1 << 15), 1 << 15, size=2048, dtype=np.int16)
    elif kind == "extremes":
        x = np.resize(np.array([-32768, 32767, -1, 0, 1, -128, 127, 32640], np.int16), 2048)
    else:  # the high byte 127 with a low byte >= 128: the edge of the two-byte split
        x = g.integers(32640, 32768, size=2048).astype(np.int16)
    Y = np.zeros(128 * 64, np.uint64)
    glc.glc_enc13_phase_a(tw.ctypes.data, x.ctypes.data, cols, Y.ctypes.data)
    xs = [int(v) for v in x[:cols]] + [0] * (2048 - cols)
    w64 = pow(w, 64, P)
    for j1 in range(128):
        wj = pow(w64, j1, P)
        for i2 in range(0, 64, 7 if kind == "uniform" else 1):
            acc, f = 0, 1
            for i1 in range(32):
                acc += xs[64 * i1 + i2] * f
                f = f * wj % P
            want = acc * pow(w, i2 * j1, P) % P
            assert int(Y[j1 * 64 + i2]) == want, (j1, i2)
