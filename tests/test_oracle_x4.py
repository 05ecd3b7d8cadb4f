"""Pins the X4 extension-field oracle (oracle/volta_oracle_x4.c).

Checks, each able to catch a plausible restatement mistake:
  * golden vectors written by the reference itself (tests/golden/
    x4_reference_vectors.json, from cuda/x4b_host_reference.cpp and
    direct_fold_reference of cuda/volta_x4b.cuh; see make_x4_golden.py);
  * the reference's unit cases of rust/volta-pcs/src/x4/ntt.rs:262-339,
    restated with independent Python big-integer arithmetic;
  * when oracle/_ref is built (this container), a live differential run
    against the reference's own header functions on random inputs.
Also pinned here: the facts about the X4 roots that the HIP path relies on
(real roots up to 2^32, equal to the base field's roots up to 2^31).
"""
import ctypes
import hashlib
import json
import pathlib
import random

import numpy as np
import pytest

P = 0xFFFF_FFFF_0000_0001
ROOT = pathlib.Path(__file__).resolve().parents[1]
GOLDEN = json.loads((ROOT / "tests/golden/x4_reference_vectors.json").read_text())
REF_LIB = ROOT / "oracle/_ref/libx4b_ref.so"


# ---- independent big-integer Fp2 (phi^2 = 7) -----------------------------------------

def f2mul(a, b):
    return ((a[0] * b[0] + 7 * a[1] * b[1]) % P, (a[0] * b[1] + a[1] * b[0]) % P)


def f2add(a, b):
    return ((a[0] + b[0]) % P, (a[1] + b[1]) % P)


def f2sub(a, b):
    return ((a[0] - b[0]) % P, (a[1] - b[1]) % P)


def f2pow(a, e):
    r = (1, 0)
    while e:
        if e & 1:
            r = f2mul(r, a)
        a = f2mul(a, a)
        e >>= 1
    return r


def f2inv(a):
    return f2pow(a, P * P - 2)


def symbol(v):  # x4/ntt.rs:262-264
    return (v % P, (3 * v + 1) % P)


# ---- roots ---------------------------------------------------------------------------

def test_x4_root_is_the_reference_value(oracle):
    assert list(oracle.x4_root_of_unity(33)) == GOLDEN["root_2_33"]


@pytest.mark.parametrize("bits", [0, 1, 2, 14, 29, 32, 33])
def test_x4_root_domains_exact_and_nested(oracle, bits):
    # x4/ntt.rs:266-279, with the order checked in big integers
    root = oracle.x4_root_of_unity(bits)
    assert f2pow(root, 1 << bits) == (1, 0)
    if bits > 0:
        assert f2pow(root, 1 << (bits - 1)) != (1, 0)
    if bits > 1:
        assert f2mul(root, root) == oracle.x4_root_of_unity(bits - 1)


def test_x4_roots_are_base_field_roots_up_to_2_31(oracle):
    # The device transform uses the base field's roots 7^((p-1)/2^b) for
    # n <= 2^31, the negated base root for n = 2^32, and an imaginary root
    # only for n = 2^33.
    for bits in range(0, 32):
        assert oracle.x4_root_of_unity(bits) == (oracle.root_of_unity(bits), 0), bits
    assert oracle.x4_root_of_unity(32) == ((P - oracle.root_of_unity(32)) % P, 0)
    r33 = oracle.x4_root_of_unity(33)
    assert r33[0] == 0 and r33[1] != 0


# ---- NTT -----------------------------------------------------------------------------

def test_x4_ntt_reference_vectors(oracle):
    g = GOLDEN["ntt32"]
    got = oracle.x4_ntt(np.array(g["coefficients"], dtype=np.uint64), g["n"])
    assert got.tolist() == g["output"]


def test_x4_ntt_matches_naive_polynomial_evaluation(oracle):
    # x4/ntt.rs:281-296: 9 coefficients, n = 32, Horner at root^k
    coeffs = [symbol(i) for i in range(9)]
    got = oracle.x4_ntt(np.array(coeffs, dtype=np.uint64), 32).tolist()
    w = oracle.x4_root_of_unity(5)
    x = (1, 0)
    for k in range(32):
        acc = (0, 0)
        for c in reversed(coeffs):
            acc = f2add(f2mul(acc, x), c)
        assert tuple(got[k]) == acc, k
        x = f2mul(x, w)


@pytest.mark.parametrize("bits", [1, 2, 3, 6, 8])
def test_x4_ntt_random_against_big_int_dft(oracle, bits):
    n = 1 << bits
    rnd = random.Random(bits)
    coeffs = [(rnd.randrange(P), rnd.randrange(P)) for _ in range(rnd.randint(1, n))]
    got = oracle.x4_ntt(np.array(coeffs, dtype=np.uint64), n).tolist()
    w = oracle.x4_root_of_unity(bits)
    for k in range(n):
        wk = f2pow(w, k)
        acc, x = (0, 0), (1, 0)
        for c in coeffs:
            acc = f2add(acc, f2mul(c, x))
            x = f2mul(x, wk)
        assert tuple(got[k]) == acc


# ---- codeword folding -------------------------------------------------------------------

def _fold_input(n):
    return np.array([[(i * 0x1_0000_01B3 + 17) % 2**64, i * i * 97 + i * 19 + 29] for i in range(n)],
                    dtype=np.uint64)


@pytest.mark.parametrize("rec", GOLDEN["folds"], ids=lambda r: "b%d_c%d_%d" % (r["bits"], r["challenge"][0] % 97,
                                                                                  r["challenge"][1] % 97))
def test_x4_fold_reference_vectors(oracle, rec):
    got = oracle.x4_fold_codeword(_fold_input(1 << rec["bits"]), rec["challenge"])
    if "output" in rec:
        assert got.tolist() == rec["output"]
    else:
        assert hashlib.sha256(np.ascontiguousarray(got).tobytes()).hexdigest() == rec["sha256"]


def test_x4_fold_against_big_int_equation(oracle):
    # scalar_fold_at of the reference's X4c host check: independent x^-1 per index
    n = 64
    rnd = random.Random(7)
    v = [(rnd.randrange(P), rnd.randrange(P)) for _ in range(n)]
    ch = (rnd.randrange(P), rnd.randrange(P))
    got = oracle.x4_fold_codeword(np.array(v, dtype=np.uint64), ch).tolist()
    w = oracle.x4_root_of_unity(6)
    half_inv = (pow(2, P - 2, P), 0)
    for j in range(n // 2):
        pos, neg = v[j], v[j + n // 2]
        even = f2mul(f2add(pos, neg), half_inv)
        odd = f2mul(f2mul(f2sub(pos, neg), half_inv), f2inv(f2pow(w, j)))
        assert tuple(got[j]) == f2add(even, f2mul(ch, odd))


def test_x4_codeword_fold_matches_coefficient_fold(oracle):
    # x4/ntt.rs:298-306: fold(encode(c)) == encode(fold_coefficients(c))
    coeffs = np.array([symbol(i + 1) for i in range(16)], dtype=np.uint64)
    ch = symbol(91)
    code = oracle.x4_ntt(coeffs, 128)
    folded = oracle.x4_fold_codeword(code, ch)
    assert folded.tolist() == oracle.x4_ntt(oracle.x4_fold_coefficients(coeffs, ch), 64).tolist()


# ---- Moebius transform ------------------------------------------------------------------

def test_mobius_preserves_every_mle_evaluation(oracle):
    # x4/ntt.rs:309-327
    table = np.array([symbol(i * i + 2) for i in range(16)], dtype=np.uint64)
    coeffs = oracle.fp2_mobius(table, inverse=False)
    point = [symbol(5), symbol(7), symbol(11), symbol(13)]
    assert oracle.mle_eval_table(table, point) == oracle.mle_eval_coefficients(coeffs, point)
    for idx in range(16):
        bpt = [(1, 0) if idx >> b & 1 else (0, 0) for b in range(4)]
        assert oracle.mle_eval_coefficients(coeffs, bpt) == tuple(table[idx].tolist())


def test_mobius_round_trip_and_big_int_inverse(oracle):
    # x4/ntt.rs:330-337; the inverse is the subset sum over x's bits
    orig = np.array([symbol(i * 17 + 3) for i in range(256)], dtype=np.uint64)
    fwd = oracle.fp2_mobius(orig, inverse=False)
    assert oracle.fp2_mobius(fwd, inverse=True).tolist() == orig.tolist()
    inv = oracle.fp2_mobius(orig, inverse=True).tolist()
    o = [tuple(x) for x in orig.tolist()]
    for x in [0, 1, 5, 128, 255, 170]:
        acc = (0, 0)
        for s in range(256):
            if s & ~x == 0:
                acc = f2add(acc, o[s])
        assert tuple(inv[x]) == acc


# ---- live differential against the reference's header (where it is built) -------------

@pytest.fixture(scope="module")
def reflib():
    if not REF_LIB.exists():
        pytest.skip("oracle/_ref not built (needs /root/reference: make -C oracle ref)")
    L = ctypes.CDLL(str(REF_LIB))
    vp = ctypes.c_void_p
    L.ref_x4_root_of_unity.argtypes = [ctypes.c_uint32, vp]
    L.ref_fp2_mul.argtypes = [vp, vp, vp]
    L.ref_fp2_inv.argtypes = [vp, vp]
    L.ref_x4_direct_fold.argtypes = [vp, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_uint64, vp]
    return L


def test_x4_roots_and_inverse_match_reference_header(oracle, reflib):
    out = np.zeros(2, np.uint64)
    for bits in range(34):
        reflib.ref_x4_root_of_unity(bits, out.ctypes.data)
        assert tuple(out.tolist()) == oracle.x4_root_of_unity(bits), bits
    rnd = random.Random(3)
    for _ in range(200):
        a = np.array([rnd.randrange(P), rnd.randrange(P)], np.uint64)
        reflib.ref_fp2_inv(a.ctypes.data, out.ctypes.data)
        assert tuple(out.tolist()) == oracle.fp2_inv(a.tolist())


@pytest.mark.parametrize("bits", [1, 4, 9, 13])
def test_x4_fold_matches_reference_header_random(oracle, reflib, bits):
    rnd = np.random.default_rng(bits)
    n = 1 << bits
    v = rnd.integers(0, P, size=(n, 2), dtype=np.uint64)
    for _ in range(3):
        ch = [int(x) for x in rnd.integers(0, P, size=2, dtype=np.uint64)]
        want = np.zeros((n // 2, 2), np.uint64)
        assert reflib.ref_x4_direct_fold(v.ctypes.data, n, ch[0], ch[1], want.ctypes.data) == 0
        assert np.array_equal(oracle.x4_fold_codeword(v, ch), want)
