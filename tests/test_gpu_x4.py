"""GPU parity of the X4 extension-field transforms through the C ABI: the Fp2
NTT with the order-2^33 root (volta_cuda_x4b_ntt_fp2 and its resident form),
codeword folding (volta_cuda_x4c_direct_fold_arena) and the Moebius inverse
(volta_cuda_fp2_mobius_inverse_inplace_device).

Checks: bit-exact against the oracle (oracle/volta_oracle_x4.c, itself pinned
to the reference's vectors) up to 2^21 points; above that, through identities
the mathematics fixes: the even/odd split NTT_2n(x)[2j] = NTT_n(x_lo + x_hi)[j],
NTT_2n(x)[2j+1] = NTT_n((x_lo - x_hi) w^i)[j]; Horner evaluation at sampled
points for the largest sizes (2^28 .. 2^33, where the order-2^32 root's sign
and the imaginary order-2^33 root take effect); fold(encode(c)) =
encode(fold_coefficients(c)) (rust/volta-pcs/src/x4/ntt.rs:298-306)."""
import ctypes
import json
import pathlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

P = 0xFFFF_FFFF_0000_0001
GOLDEN = json.loads((pathlib.Path(__file__).resolve().parent / "golden/x4_reference_vectors.json").read_text())


def rand_fp2(seed, n):
    return np.random.Generator(np.random.PCG64(seed)).integers(0, P, size=(n, 2), dtype=np.uint64)


def f2mul(a, b):
    return ((a[0] * b[0] + 7 * a[1] * b[1]) % P, (a[0] * b[1] + a[1] * b[0]) % P)


def f2add(a, b):
    return ((a[0] + b[0]) % P, (a[1] + b[1]) % P)


def horner(coeffs, x):
    acc = (0, 0)
    for c in reversed(coeffs):
        acc = f2add(f2mul(acc, x), c)
    return acc


def sample_indices(n, seed, count=48):
    rnd = np.random.Generator(np.random.PCG64(seed))
    fixed = [0, 1, 2, 3, n // 2 - 1, n // 2, n // 2 + 1, n - 2, n - 1]
    if n > 1 << 31:
        fixed += [(1 << 31) - 1, 1 << 31, (1 << 31) + 1, (1 << 31) + 3]
    picks = [int(v) for v in rnd.integers(0, n, size=count)]
    return sorted(set(i for i in fixed + picks if 0 <= i < n))


# ---- NTT: oracle parity -----------------------------------------------------------------

@pytest.mark.parametrize("bits,length", [
    (1, 1), (1, 2), (2, 3), (3, 8), (5, 1), (7, 100), (11, 2048), (12, 4096), (12, 9),
    (13, 5000), (14, 1), (16, 65536), (17, 3), (20, 700001), (21, 1 << 21),
    # just past k n / A, where the first pass reads k + 1 of its A step-1 inputs
    # (A = 16 at 2^16, 8 at 2^18)
    (16, 4097), (16, 8193), (16, 16385), (16, 20481), (18, 32769), (18, 65537), (18, 98305),
])
def test_x4_ntt_matches_oracle(backend, oracle, bits, length):
    n = 1 << bits
    x = rand_fp2(bits * 1000 + length, length)
    got = backend.x4b_ntt_fp2(x, n)
    assert np.array_equal(got, oracle.x4_ntt(x, n))


def test_x4_ntt_reference_vectors(backend):
    g = GOLDEN["ntt32"]
    got = backend.x4b_ntt_fp2(np.array(g["coefficients"], dtype=np.uint64), g["n"])
    assert got.tolist() == g["output"]


def test_x4_ntt_resident_matches_host_form(backend):
    from volta_mi355x import FP2
    n, length = 1 << 15, 12345
    x = rand_fp2(5, length)
    d = backend.alloc_device(length + 3, FP2)
    backend.upload_into(d, 3, x.reshape(-1).view(FP2))
    out = backend.alloc_device(n + 1, FP2)
    backend.x4_ntt_fp2_device(d, length, n, out, in_offset=3, out_offset=1)
    got = backend.download_device(out, 1, n).view(np.uint64).reshape(n, 2)
    # the input region is left unchanged
    assert np.array_equal(backend.download_device(d, 3, length).view(np.uint64).reshape(length, 2), x)
    backend.free_device(d)
    backend.free_device(out)
    assert np.array_equal(got, backend.x4b_ntt_fp2(x, n))


# ---- NTT: sizes above the oracle's, by the even/odd split -------------------------------

def _split_inputs(oracle, x):
    """(x_lo + x_hi, (x_lo - x_hi) w^i) for the 2n-point root w, componentwise."""
    n = x.shape[0] // 2
    lo, hi = x[:n], x[n:]
    w = oracle.ntt_twiddles(2 * n)  # w^0 .. w^(n-1), the base root = the X4 root below 2^32
    even = np.stack([oracle.fp_add_vec(lo[:, k].copy(), hi[:, k].copy()) for k in range(2)], axis=1)
    odd = np.stack([oracle.fp_mul_vec(oracle.fp_sub_vec(lo[:, k].copy(), hi[:, k].copy()), w) for k in range(2)],
                   axis=1)
    return even, odd


@pytest.mark.parametrize("bits", [22, 23, 24, 26])
def test_x4_ntt_even_odd_split(backend, oracle, bits):
    from volta_mi355x import FP2
    n = 1 << bits
    x = rand_fp2(bits, n)
    even, odd = _split_inputs(oracle, x)
    dx, de, do = (backend.upload_device(a, FP2) for a in (x, even, odd))
    full = backend.x4_ntt_fp2_device(dx, n, n)
    he = backend.x4_ntt_fp2_device(de, n // 2, n // 2)
    ho = backend.x4_ntt_fp2_device(do, n // 2, n // 2)
    got = backend.download_device(full).view(np.uint64).reshape(n, 2)
    want_e = backend.download_device(he).view(np.uint64).reshape(n // 2, 2)
    want_o = backend.download_device(ho).view(np.uint64).reshape(n // 2, 2)
    for b in (dx, de, do, full, he, ho):
        backend.free_device(b)
    if bits == 22:  # anchor the chain: the half-size transforms against the oracle
        assert np.array_equal(want_e, oracle.x4_ntt(even, n // 2))
    assert np.array_equal(got[0::2], want_e)
    assert np.array_equal(got[1::2], want_o)


# ---- NTT: the largest sizes, sampled -----------------------------------------------------

@pytest.mark.parametrize("bits,length", [(28, 4096), (30, 1000), (31, 4096), (32, 4096), (33, 4096)])
def test_x4_ntt_huge_sampled(backend, oracle, bits, length):
    """All P passes at full size, with a ragged coefficient tail; 2^32 and 2^33
    use the order-2^32 root (-b_32) and the imaginary order-2^33 root."""
    from volta_mi355x import FP2
    n = 1 << bits
    x = rand_fp2(bits + 7, length)
    d = backend.upload_device(x, FP2)
    out = backend.x4_ntt_fp2_device(d, length, n)
    coeffs = [tuple(int(v) for v in row) for row in x.tolist()]
    w = oracle.x4_root_of_unity(bits)
    try:
        for j in sample_indices(n, bits):
            got = tuple(int(v) for v in backend.download_device(out, j, 1).view(np.uint64))
            assert got == horner(coeffs, oracle.fp2_pow(w, j)), j
    finally:
        backend.free_device(d)
        backend.free_device(out)


# ---- codeword fold ---------------------------------------------------------------------------

def _fold_on_device(backend, values, challenge, in_off_elems=0, gap=0):
    from volta_mi355x import FP2
    n = values.shape[0]
    arena = backend.alloc_device(in_off_elems + n + gap + n // 2, FP2)
    backend.upload_into(arena, in_off_elems, values.reshape(-1).view(FP2))
    out_off = in_off_elems + n + gap
    backend.x4c_direct_fold_arena_into_arena(arena, in_off_elems * 16, n, out_off * 16, challenge)
    got = backend.download_device(arena, out_off, n // 2).view(np.uint64).reshape(n // 2, 2)
    backend.free_device(arena)
    return got


def _fold_input(n):
    return np.array([[(i * 0x1_0000_01B3 + 17) % 2**64, i * i * 97 + i * 19 + 29] for i in range(n)], dtype=np.uint64)


@pytest.mark.parametrize("rec", [r for r in GOLDEN["folds"] if "output" in r],
                         ids=lambda r: "b%d_c%d" % (r["bits"], r["challenge"][0] % 1000))
def test_x4_fold_reference_vectors(backend, rec):
    got = _fold_on_device(backend, _fold_input(1 << rec["bits"]), rec["challenge"])
    assert got.tolist() == rec["output"]


@pytest.mark.parametrize("bits,in_off,gap", [(1, 0, 0), (2, 1, 0), (5, 0, 3), (9, 2, 1), (13, 0, 0), (17, 5, 0),
                                             (20, 0, 7), (22, 0, 0)])
def test_x4_fold_matches_oracle(backend, oracle, bits, in_off, gap):
    n = 1 << bits
    v = rand_fp2(bits * 3 + in_off, n)
    for ch in [(0, 0), (1, 0), (P - 1, P - 2), tuple(int(c) for c in rand_fp2(bits, 1)[0])]:
        got = _fold_on_device(backend, v, ch, in_off, gap)
        assert np.array_equal(got, oracle.x4_fold_codeword(v, ch)), ch


@pytest.mark.parametrize("bits,length", [(20, 1 << 17), (28, 4096), (32, 4096), (33, 4096)])
def test_x4_fold_of_encode_is_encode_of_fold(backend, oracle, bits, length):
    """fold(NTT_n(c)) = NTT_(n/2)(c[2i] + ch c[2i+1]) (x4/ntt.rs:298-306), with
    the codeword built in place by the resident NTT; sampled above 2^20."""
    from volta_mi355x import FP2
    n = 1 << bits
    c = rand_fp2(bits + 11, length)
    ch = tuple(int(v) for v in rand_fp2(bits + 12, 1)[0])
    d = backend.upload_device(c, FP2)
    arena = backend.alloc_device(n + n // 2, FP2)
    try:
        backend.x4_ntt_fp2_device(d, length, n, arena)
        backend.x4c_direct_fold_arena_into_arena(arena, 0, n, n * 16, ch)
        fc = oracle.x4_fold_coefficients(c, ch)
        if bits <= 20:
            got = backend.download_device(arena, n, n // 2).view(np.uint64).reshape(n // 2, 2)
            assert np.array_equal(got, oracle.x4_ntt(fc, n // 2))
        else:
            fcl = [tuple(int(v) for v in row) for row in fc.tolist()]
            w = oracle.x4_root_of_unity(bits - 1)
            for j in sample_indices(n // 2, bits):
                got = tuple(int(v) for v in backend.download_device(arena, n + j, 1).view(np.uint64))
                assert got == horner(fcl, oracle.fp2_pow(w, j)), j
    finally:
        backend.free_device(d)
        backend.free_device(arena)


def test_x4_fold_pinned_tiles_match_oracle(backend, oracle):
    """A codeword folded tile by tile from pinned host memory
    (volta_cuda_x4c_direct_fold_pinned_tile) equals the whole fold; pinned
    uploads land byte-exact (volta_cuda_x4c_upload_pinned)."""
    from volta_mi355x import FP2
    bits, tile = 14, 1000  # tiles of 1000 outputs, the last one short
    n, half = 1 << bits, 1 << (bits - 1)
    v = rand_fp2(77, n)
    ch = tuple(int(c) for c in rand_fp2(78, 1)[0])
    want = oracle.x4_fold_codeword(v, ch)
    out_off, scratch_off = 0, half * 16
    arena = backend.alloc_device(half + 2 * tile, FP2)
    pin = backend.pinned_alloc(2 * tile * 16 * 2)  # two tile slots, used alternately
    launches0 = backend.get_stats()["x4c_kernel_launches"]
    try:
        for k, start in enumerate(range(0, half, tile)):
            cnt = min(tile, half - start)
            slot = (k % 2) * 2 * tile * 16
            backend.pinned_write(pin, slot, np.concatenate([v[start:start + cnt], v[half + start:half + start + cnt]]))
            backend.x4c_direct_fold_pinned_tile(pin, slot, arena, out_off, scratch_off, n, start, cnt, ch)
        got = backend.download_device(arena, 0, half).view(np.uint64).reshape(half, 2)
        assert np.array_equal(got, want)
        assert backend.get_stats()["x4c_kernel_launches"] - launches0 == -(-half // tile)
        # the plain pinned upload
        backend.pinned_write(pin, 0, v[:tile])
        backend.x4c_upload_pinned(pin, 0, arena, scratch_off, tile * 16)
        back = backend.download_device(arena, half, tile).view(np.uint64).reshape(tile, 2)
        assert np.array_equal(back, v[:tile])
    finally:
        backend.pinned_wait_ready(pin)
        backend.pinned_free(pin)
        backend.free_device(arena)


def test_x4_fold_pinned_tile_errors(backend):
    from volta_mi355x import FP2
    lib, raw = backend.lib, backend.raw
    arena = backend.alloc_device(64, FP2)
    pin = backend.pinned_alloc(1024)
    f = lib.volta_cuda_x4c_direct_fold_pinned_tile
    try:
        assert f(raw, pin, 0, arena.id, 0, 512, 64, 0, 0, 1, 1) != 0  # no outputs
        assert "invalid X4c pinned direct-fold geometry" in backend.last_error()
        assert f(raw, pin, 0, arena.id, 0, 512, 64, 30, 3, 1, 1) != 0  # past n/2
        assert "invalid X4c pinned direct-fold geometry" in backend.last_error()
        assert f(raw, pin, 8, arena.id, 0, 512, 64, 0, 4, 1, 1) != 0
        assert "misaligned" in backend.last_error()
        assert f(raw, pin, 0, arena.id, 0, 256, 64, 0, 4, 1, 1) != 0  # scratch inside the output
        assert "overlap" in backend.last_error()
        assert f(raw, pin, 0, arena.id, 0, 512, 128, 0, 33, 1, 1) != 0  # 1056-byte tile, 1024-byte buffer
        assert "out of bounds" in backend.last_error()
        assert lib.volta_cuda_x4c_upload_pinned(raw, pin, 1000, arena.id, 0, 100) != 0
        assert "out of bounds" in backend.last_error()
        assert lib.volta_cuda_x4c_upload_pinned(raw, 12345, 0, arena.id, 0, 16) != 0
        assert "pinned buffer id" in backend.last_error()
    finally:
        backend.pinned_free(pin)
        backend.free_device(arena)


# ---- Moebius inverse --------------------------------------------------------------------------

@pytest.mark.parametrize("bits,off", [(0, 0), (1, 0), (2, 1), (5, 0), (11, 3), (12, 0), (13, 0), (14, 2), (17, 0),
                                      (22, 0), (23, 1)])
def test_mobius_inverse_matches_oracle(backend, oracle, bits, off):
    from volta_mi355x import FP2
    n = 1 << bits
    v = rand_fp2(bits + 100, n)
    d = backend.alloc_device(off + n + 2, FP2)
    guard = rand_fp2(7, off + n + 2)
    backend.upload_into(d, 0, guard.reshape(-1).view(FP2))
    backend.upload_into(d, off, v.reshape(-1).view(FP2))
    backend.fp2_mobius_inverse_inplace_device(d, off, n)
    got = backend.download_device(d).view(np.uint64).reshape(-1, 2)
    backend.free_device(d)
    assert np.array_equal(got[off:off + n], oracle.fp2_mobius(v, inverse=True))
    # neighbours are untouched
    assert np.array_equal(got[:off], guard[:off]) and np.array_equal(got[off + n:], guard[off + n:])


# ---- geometry errors and stats ---------------------------------------------------------------

def test_x4_geometry_errors(backend):
    from volta_mi355x import FP2
    lib, raw = backend.lib, backend.raw
    x = np.zeros((4, 2), np.uint64)
    out = np.zeros((8, 2), np.uint64)
    for length, n in [(0, 8), (9, 8), (1, 1), (3, 12), (1, 1 << 34)]:
        assert lib.volta_cuda_x4b_ntt_fp2(raw, x.ctypes.data, length, n, out.ctypes.data) != 0
        assert "invalid X4b Fp2 NTT geometry" in backend.last_error()
    assert lib.volta_cuda_x4b_ntt_fp2(raw, None, 1, 8, out.ctypes.data) != 0
    arena = backend.alloc_device(64, FP2)
    fold = lib.volta_cuda_x4c_direct_fold_arena
    assert fold(raw, arena.id, 0, 3, 512, 1, 1) != 0  # not a power of two
    assert "invalid X4c arena direct-fold geometry" in backend.last_error()
    assert fold(raw, arena.id, 0, 8, 512, P, 0) != 0  # challenge not canonical
    assert "invalid X4c arena direct-fold geometry" in backend.last_error()
    assert fold(raw, arena.id, 8, 8, 512, 1, 1) != 0
    assert "misaligned" in backend.last_error()
    assert fold(raw, arena.id, 0, 8, 64, 1, 1) != 0  # output overlaps the input
    assert "overlap" in backend.last_error()
    assert fold(raw, arena.id, 0, 64, 1024, 1, 1) != 0  # output past the arena
    assert "out of bounds" in backend.last_error()
    assert lib.volta_cuda_fp2_mobius_inverse_inplace_device(raw, arena.id, 0, 3) != 0
    assert "invalid resident Fp2 Mobius inverse" in backend.last_error()
    assert lib.volta_cuda_fp2_mobius_inverse_inplace_device(raw, arena.id, 1, 64) != 0
    assert "out of bounds" in backend.last_error()
    d = backend.alloc_device(16, FP2)
    assert lib.volta_mi355x_x4_ntt_fp2_device(raw, d.id, 0, 16, 16, d.id, 0) != 0
    assert "overlap" in backend.last_error()
    for b in (arena, d):
        backend.free_device(b)


def test_x4_ntt_stats_accounting():
    """One host X4 NTT: the coefficients (plus first-use tables) up, the
    codeword down, the tail counted as zeroed, one OP_PCS_NTT call."""
    from volta_mi355x import Backend
    with Backend() as b:
        x = rand_fp2(1, 100)
        b.x4b_ntt_fp2(x, 1 << 10)  # warm: builds the tables
        b.reset_stats()
        b.x4b_ntt_fp2(x, 1 << 10)
        s = b.get_stats()
        assert s["calls"]["pcs_ntt"] == 1
        assert s["h2d_bytes"] == 100 * 16
        assert s["d2h_bytes"] == (1 << 10) * 16
        assert s["device_zeroed_bytes"] == ((1 << 10) - 100) * 16
        assert s["kernel_ns"]["pcs_ntt"] > 0
