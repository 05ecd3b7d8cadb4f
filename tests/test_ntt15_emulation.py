"""The one-pass 2^15-point transform (volta-zk_amd/csrc/ntt15.hip), its phases
built for the host from the same header (ntt15.hpp, in libgl64_check.so) and
run thread by thread between the kernel's barriers, against the oracle's
transform of the zero-tailed rows.  The emulation poisons the exchange buffer
before every write round and checks guard words around the LDS image and its
table after every row, so a read of a word that the round did not write, or
a write outside the buffer, fails here on the CPU.  CPU only."""
import ctypes
import pathlib

import numpy as np
import pytest

import oracle

LIB = pathlib.Path(__file__).resolve().parent.parent / "volta-zk_amd" / "libgl64_check.so"
N = 1 << 15
P = 0xFFFF_FFFF_0000_0001


@pytest.fixture(scope="module")
def glc():
    if not LIB.exists():
        pytest.fail("libgl64_check.so missing: run volta-zk_amd/build.py (or __graft_entry__.build())")
    L = ctypes.CDLL(str(LIB))
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    L.glc_ntt15_u64.restype = ctypes.c_int
    L.glc_ntt15_u64.argtypes = [vp, vp, sz, sz, sz, sz, vp]
    L.glc_ntt15_msg.restype = ctypes.c_int
    L.glc_ntt15_msg.argtypes = [vp, vp, vp, sz, sz, sz, sz, vp]
    return L


def _p(a):
    return a.ctypes.data


@pytest.fixture(scope="module")
def fwd():
    return np.ascontiguousarray(oracle.ntt_twiddles(N))


def _field(rng, shape):
    x = rng.integers(0, 1 << 63, size=shape, dtype=np.uint64) * np.uint64(2)
    x += rng.integers(0, 2, size=shape, dtype=np.uint64)
    return np.where(x >= np.uint64(P), x - np.uint64(P), x)


@pytest.mark.parametrize("length,stride", [(1, 1), (2048, 2048), (3000, 3001), (4096, 4096), (4097, 5000),
                                           (8192, 8192), (8193, 8193), (16896, 16896), (32768, 32768)])
def test_u64_rows_match_the_oracle(glc, fwd, length, stride):
    rng = np.random.default_rng(length)
    rows, blocks = 3, 2  # block 0 takes rows 0 and 2: the row loop and its prefetch run
    src = _field(rng, (rows, stride))
    want = np.zeros((rows, N), dtype=np.uint64)
    want[:, :length] = src[:, :length]
    want = oracle.ntt_forward_batch(want)
    got = np.zeros((rows, N), dtype=np.uint64)
    rc = glc.glc_ntt15_u64(_p(fwd), _p(src), stride, length, rows, blocks, _p(got))
    assert rc == 0
    assert (got == want).all()


def test_u64_rows_edge_values(glc, fwd):
    vals = np.array([0, 1, P - 1, P - 2, 0xFFFFFFFF, 1 << 32, (1 << 63), P - (1 << 32)], dtype=np.uint64)
    src = np.resize(vals, (2, 4096)).astype(np.uint64)
    want = np.zeros((2, N), dtype=np.uint64)
    want[:, :4096] = src
    got = np.zeros((2, N), dtype=np.uint64)
    assert glc.glc_ntt15_u64(_p(fwd), _p(src), 4096, 4096, 2, 1, _p(got)) == 0
    assert (got == oracle.ntt_forward_batch(want)).all()


def test_u64_rows_refused_past_n(glc, fwd):
    src = np.zeros((1, N + 1), dtype=np.uint64)
    got = np.zeros((1, N), dtype=np.uint64)
    assert glc.glc_ntt15_u64(_p(fwd), _p(src), N + 1, N + 1, 1, 1, _p(got)) == 1


@pytest.mark.parametrize("cols,pad", [(8192, 0), (8192, 512), (8192, 1024), (4096, 0), (4096, 512)])
def test_message_rows_match_the_oracle(glc, fwd, cols, pad):
    rng = np.random.default_rng(cols + pad)
    rows, blocks = 3, 2
    w = rng.integers(-32768, 32768, size=(rows, cols), dtype=np.int16)
    w[0, :4] = [-32768, 32767, -1, 0]
    pads = _field(rng, (rows, max(pad, 1)))
    msgs = oracle.pcs_messages(w.reshape(-1), pads.reshape(-1) if pad else None, rows, cols, pad, N)
    want = oracle.ntt_forward_batch(msgs.reshape(rows, N))
    got = np.zeros((rows, N), dtype=np.uint64)
    rc = glc.glc_ntt15_msg(_p(fwd), _p(w), _p(pads), cols, pad, rows, blocks, _p(got))
    assert rc == 0
    assert (got == want).all()


# ---- the one-pass 2^13 and 2^14 transforms of rows that may be dense (ntt_rr.hpp) ---

N13 = 1 << 13


@pytest.fixture(scope="module")
def fwd13():
    return np.ascontiguousarray(oracle.ntt_twiddles(N13))


@pytest.mark.parametrize("length,stride", [(1, 1), (2048, 2048), (2049, 2100), (4096, 4096), (5000, 5000),
                                           (8192, 8192)])
def test_ntt13_dense_rows_match_the_oracle(glc, fwd13, length, stride):
    glc.glc_ntt13r_u64.restype = ctypes.c_int
    glc.glc_ntt13r_u64.argtypes = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_size_t] * 4 + [ctypes.c_void_p]
    rng = np.random.default_rng(length + 13)
    rows, blocks = 5, 2
    src = _field(rng, (rows, stride))
    edge = np.array([0, 1, P - 1, P - 2], dtype=np.uint64)[:stride]
    src[0, :edge.size] = edge
    want = np.zeros((rows, N13), dtype=np.uint64)
    want[:, :length] = src[:, :length]
    want = oracle.ntt_forward_batch(want)
    got = np.zeros((rows, N13), dtype=np.uint64)
    assert glc.glc_ntt13r_u64(_p(fwd13), _p(src), stride, length, rows, blocks, _p(got)) == 0
    assert (got == want).all()


N14 = 1 << 14


@pytest.fixture(scope="module")
def fwd14():
    return np.ascontiguousarray(oracle.ntt_twiddles(N14))


@pytest.mark.parametrize("length,stride", [(1, 1), (4096, 4096), (4097, 4100), (8192, 8192), (9000, 9000),
                                           (16384, 16384)])
def test_ntt14_rows_match_the_oracle(glc, fwd14, length, stride):
    glc.glc_ntt14r_u64.restype = ctypes.c_int
    glc.glc_ntt14r_u64.argtypes = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_size_t] * 4 + [ctypes.c_void_p]
    rng = np.random.default_rng(length + 14)
    rows, blocks = 5, 2
    src = _field(rng, (rows, stride))
    edge = np.array([0, 1, P - 1, P - 2], dtype=np.uint64)[:stride]
    src[0, :edge.size] = edge
    want = np.zeros((rows, N14), dtype=np.uint64)
    want[:, :length] = src[:, :length]
    want = oracle.ntt_forward_batch(want)
    got = np.zeros((rows, N14), dtype=np.uint64)
    assert glc.glc_ntt14r_u64(_p(fwd14), _p(src), stride, length, rows, blocks, _p(got)) == 0
    assert (got == want).all()


@pytest.mark.parametrize("log_n", [13, 14])
def test_rows_read_in_full_with_zero_tails(glc, fwd13, fwd14, log_n):
    """Rows passed at full length (the kernels read them whole) whose values
    are zero from 8 M on (M = n / 32: 2048 at 2^13, 4096 at 2^14), as message
    rows are: a wave whose inputs are all zero there runs stage A's first two
    stages as copies.  Row 0 has that tail zero (every wave copies), row 1 one
    nonzero value at 8 M + 5 (only the wave holding it runs them in full), row 2
    is dense, row 3 nonzero only at n - 1; every row against the oracle, and
    the waves of each kind counted."""
    n = 1 << log_n
    fn = glc.glc_ntt13r_u64 if log_n == 13 else glc.glc_ntt14r_u64
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_size_t] * 4 + [ctypes.c_void_p]
    glc.glc_rr_wave_counts.restype = None
    glc.glc_rr_wave_counts.argtypes = [ctypes.POINTER(ctypes.c_long), ctypes.POINTER(ctypes.c_long), ctypes.c_int]
    m8 = 8 * (n // 32)
    rng = np.random.default_rng(log_n + 100)
    src = np.zeros((4, n), dtype=np.uint64)
    src[:, :m8] = _field(rng, (4, m8))
    src[0, :4] = np.array([0, 1, P - 1, P - 2], dtype=np.uint64)
    src[1, m8 + 5] = P - 1
    src[2] = _field(rng, (1, n))[0]
    src[3, n - 1] = 12345
    full, copy = ctypes.c_long(), ctypes.c_long()
    glc.glc_rr_wave_counts(ctypes.byref(full), ctypes.byref(copy), 1)
    got = np.zeros((4, n), dtype=np.uint64)
    assert fn(_p(fwd13 if log_n == 13 else fwd14), _p(src), n, n, 4, 2, _p(got)) == 0
    assert (got == oracle.ntt_forward_batch(src)).all()
    glc.glc_rr_wave_counts(ctypes.byref(full), ctypes.byref(copy), 1)
    waves = (n // 32) // 64
    assert (full.value, copy.value) == (1 + waves + 1, waves + 2 * (waves - 1))
