"""Phase B of the n = 2^13 i16 encode (volta-zk_amd/csrc/enc13_phase_b.hpp): the
64-point DFT over i2 of one row of Y, as the first radix-2 stage's sums and
differences (phase A's stores) followed by one 32-point DFT of powers-of-two
twiddles per output parity.  Built for the host
from the same header (libgl64_check.so) and checked against the defining sum
X[j2] = sum_{i2 < 64} Y[i2] w64^(i2 j2), w64 = w^128 for the 2^13-th root w
the reference's transform uses (rust/volta-pcs/src/ntt.rs:9-12).  CPU only."""
import ctypes
import pathlib
import random

import pytest

P = 0xFFFF_FFFF_0000_0001
LIB = pathlib.Path(__file__).resolve().parent.parent / "volta-zk_amd" / "libgl64_check.so"
W64 = pow(pow(7, (P - 1) >> 13, P), 128, P)


@pytest.fixture(scope="module")
def glc():
    if not LIB.exists():
        pytest.fail("libgl64_check.so missing: run volta-zk_amd/build.py (or __graft_entry__.build())")
    L = ctypes.CDLL(str(LIB))
    L.glc_enc13_phase_b.restype = None
    L.glc_enc13_phase_b.argtypes = [ctypes.POINTER(ctypes.c_uint64), ctypes.c_int, ctypes.POINTER(ctypes.c_uint64)]
    return L


def _rows():
    rnd = random.Random(13)
    yield "uniform", [rnd.randrange(P) for _ in range(64)]
    yield "zeros", [0] * 64
    yield "p-1", [P - 1] * 64
    yield "one-hot", [1 if i == 37 else 0 for i in range(64)]
    # equal halves: every D[q] is 0
    half = [rnd.randrange(P) for _ in range(32)]
    yield "equal halves", half + half
    # opposite halves: every S[q] is 0
    yield "opposite halves", half + [(P - v) % P for v in half]
    yield "top band", [P - 1 - rnd.randrange(1 << 33) for _ in range(64)]
    yield "small", [rnd.randrange(1 << 20) for _ in range(64)]


@pytest.mark.parametrize("H", [0, 1])
@pytest.mark.parametrize("name,y", list(_rows()), ids=[n for n, _ in _rows()])
def test_phase_b_matches_the_defining_sum(glc, H, name, y):
    yin = (ctypes.c_uint64 * 64)(*y)
    out = (ctypes.c_uint64 * 32)()
    glc.glc_enc13_phase_b(yin, H, out)
    for k in range(32):
        j2 = 2 * k + H
        want = sum(y[i2] * pow(W64, i2 * j2, P) for i2 in range(64)) % P
        assert out[k] == want, (name, H, k)


def test_w64_is_the_power_of_two_the_kernel_shifts_by():
    assert W64 == pow(2, 39, P)
