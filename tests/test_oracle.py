"""Pins the CPU oracle before it is trusted as the checker.

Each check is chosen so a plausible restatement mistake (dropped carry term,
wrong twiddle index, transposed operand, wrong word order) fails it:
  * reference-recorded checksums of the reference's own arithmetic runs
    (benchmarks/results/p7-gpu-pcs-arithmetic[-quick]-2026-07-11-366ec4a.json,
    p7-gpu-roofline[-quick]-2026-07-11-a43d105.json);
  * the reference's unit cases (rust/volta-field/src/lib.rs:297-351,
    rust/volta-pcs/src/ntt.rs:78-121) restated;
  * Python big-integer arithmetic and brute-force DFTs;
  * the ChaCha8 KAT of rust/volta-accel/src/lib.rs:7517-7528 and the
    published all-zero-key ChaCha8 keystream.
"""
import random

import numpy as np
import pytest

import spike_inputs as spike

P = 0xFFFF_FFFF_0000_0001
EPS = 0xFFFF_FFFF
MASK64 = (1 << 64) - 1


# ---- field ------------------------------------------------------------------

def test_field_differential_against_big_ints(oracle):
    rnd = random.Random(0xB0)
    a = np.array([rnd.randrange(P) for _ in range(20000)], dtype=np.uint64)
    b = np.array([rnd.randrange(P) for _ in range(20000)], dtype=np.uint64)
    # include the boundary values
    a[:4] = [0, 1, P - 1, P - 2]
    b[:4] = [P - 1, P - 1, P - 1, 1]
    mul, add, sub = oracle.fp_mul_vec(a, b), oracle.fp_add_vec(a, b), oracle.fp_sub_vec(a, b)
    for x, y, m, s, d in zip(a.tolist(), b.tolist(), mul.tolist(), add.tolist(), sub.tolist()):
        assert m == x * y % P
        assert s == (x + y) % P
        assert d == (x - y) % P


def test_field_edge_cases(oracle):
    # rust/volta-field/src/lib.rs:309-320
    assert oracle.fp_mul(P - 1, P - 1) == 1
    assert oracle.fp_add(P - 1, 1) == 0
    assert oracle.fp_sub(0, 1) == P - 1
    assert oracle.fp_new(MASK64) == MASK64 - P
    assert oracle.fp_pow(2, 64) == EPS
    assert oracle.fp_pow(2, 96) == P - 1
    assert oracle.fp_from_i64(-5) == oracle.fp_sub(0, 5)
    assert oracle.fp_from_i64(-32768) == P - 32768
    assert oracle.fp_from_i64(32767) == 32767
    assert oracle.fp_neg(0) == 0 and oracle.fp_neg(3) == P - 3


def test_inverse_and_non_residue(oracle):
    rnd = random.Random(1)
    for _ in range(200):
        a = rnd.randrange(1, P)
        assert oracle.fp_mul(a, oracle.fp_inv(a)) == 1
    # lib.rs:331-335: 7 is a quadratic non-residue
    assert oracle.fp_pow(7, (P - 1) // 2) == P - 1


def _fp2_mul_ref(a, b):
    return ((a[0] * b[0] + 7 * a[1] * b[1]) % P, (a[0] * b[1] + a[1] * b[0]) % P)


def test_fp2_against_big_ints(oracle):
    rnd = random.Random(2)
    for _ in range(500):
        a = (rnd.randrange(P), rnd.randrange(P))
        b = (rnd.randrange(P), rnd.randrange(P))
        x = rnd.randrange(P)
        assert oracle.fp2_mul(a, b) == _fp2_mul_ref(a, b)
        assert oracle.fp2_add(a, b) == ((a[0] + b[0]) % P, (a[1] + b[1]) % P)
        assert oracle.fp2_mul_base(a, x) == (a[0] * x % P, a[1] * x % P)


def test_fp2_powers_start_at_c(oracle):
    # ligero.rs:772-778: c^1 .. c^rows
    c = (123456789, 987654321)
    got = oracle.fp2_powers(c, 5)
    acc = (1, 0)
    for k in range(5):
        acc = _fp2_mul_ref(acc, c)
        assert tuple(int(v) for v in got[k]) == acc


# ---- NTT ------------------------------------------------------------------------

def _naive_dft(a, w):
    n = len(a)
    return [sum(a[i] * pow(w, i * j, P) for i in range(n)) % P for j in range(n)]


def test_root_has_exact_order(oracle):
    # ntt.rs:78-87
    for bits in (1, 4, 15, 32):
        w = oracle.root_of_unity(bits)
        assert pow(w, 1 << (bits - 1), P) == P - 1
        assert pow(w, 1 << bits, P) == 1
    assert oracle.root_of_unity(5) == pow(7, (P - 1) >> 5, P)


def test_ntt_matches_naive_dft_n16(oracle):
    # ntt.rs:89-104: a_i = i^2 + 3
    a = np.array([i * i + 3 for i in range(16)], dtype=np.uint64)
    got = oracle.ntt_forward_batch(a.reshape(1, 16))[0]
    assert got.tolist() == _naive_dft(a.tolist(), oracle.root_of_unity(4))


@pytest.mark.parametrize("bits", [1, 2, 3, 5, 7, 8])
def test_ntt_matches_naive_dft_random(oracle, bits):
    n = 1 << bits
    rnd = random.Random(bits)
    a = [rnd.randrange(P) for _ in range(n)]
    got = oracle.ntt_forward_batch(np.array([a], dtype=np.uint64))[0]
    assert got.tolist() == _naive_dft(a, pow(7, (P - 1) >> bits, P))


def test_encode_is_polynomial_evaluation(oracle):
    # ntt.rs:106-121: codeword[j] = poly(w^j) for a zero-padded message
    msg = [7 * i + 1 for i in range(5)]
    code = oracle.ntt_encode_batch(np.array([msg], dtype=np.uint64), 32)[0]
    w = oracle.root_of_unity(5)
    for j in (0, 1, 17, 31):
        x = pow(w, j, P)
        acc = 0
        for c in reversed(msg):
            acc = (acc * x + c) % P
        assert int(code[j]) == acc


def test_inverse_ntt_round_trip_and_naive(oracle):
    rnd = random.Random(9)
    a = np.array([[rnd.randrange(P) for _ in range(64)] for _ in range(3)], dtype=np.uint64)
    fwd = oracle.ntt_forward_batch(a)
    assert (oracle.ntt_inverse_batch(fwd) == a).all()
    # a_i = n^-1 sum_j A_j w^-ij
    n = 64
    w_inv = pow(pow(7, (P - 1) >> 6, P), P - 2, P)
    n_inv = pow(n, P - 2, P)
    A = fwd[0].tolist()
    naive = [n_inv * x % P for x in _naive_dft(A, w_inv)]
    assert naive == a[0].tolist()


@pytest.mark.parametrize("rows,bits,msg_len,expected", spike.NTT_GOLDEN)
def test_ntt_reference_checksums(oracle, rows, bits, msg_len, expected):
    out = oracle.ntt_forward_batch(spike.ntt_input(rows, bits, msg_len))
    assert oracle.fnv(out) == expected


@pytest.mark.parametrize("rows,cols,expected", spike.COMBINE_GOLDEN)
def test_combination_reference_checksums(oracle, rows, cols, expected):
    w, q, c = spike.combine_inputs(rows, cols)
    coeffs = np.concatenate([q, c]).reshape(2 * rows, 2)
    u = oracle.combine_rows_fp(w, coeffs, 2)
    assert spike.combine_checksum(oracle.fnv, u[0], u[1]) == expected


def test_combination_brute_force_i16_with_pads(oracle):
    rnd = random.Random(5)
    rows, cols, pad, comb = 5, 6, 3, 2
    w = np.array([rnd.randrange(-32768, 32768) for _ in range(rows * cols)], dtype=np.int16)
    pads = np.array([rnd.randrange(P) for _ in range(rows * pad)], dtype=np.uint64)
    co = np.array([[rnd.randrange(P), rnd.randrange(P)] for _ in range(comb * rows)], dtype=np.uint64)
    got = oracle.pcs_combine_rows(w, pads, co, rows, cols, pad, comb)
    for k in range(comb):
        for j in range(cols + pad):
            s0 = s1 = 0
            for i in range(rows):
                x = int(w[i * cols + j]) % P if j < cols else int(pads[i * pad + j - cols])
                s0 += int(co[k * rows + i, 0]) * x
                s1 += int(co[k * rows + i, 1]) * x
            assert (int(got[k, j, 0]), int(got[k, j, 1])) == (s0 % P, s1 % P)


def test_messages_lift_and_layout(oracle):
    w = np.array([0, -1, 32767, -32768], dtype=np.int16)
    pads = np.array([11, 12], dtype=np.uint64)
    m = oracle.pcs_messages(w, pads, 2, 2, 1, 4)
    assert m.tolist() == [[0, P - 1, 11, 0], [32767, P - 32768, 12, 0]]


@pytest.mark.parametrize("log2,expected", spike.FP2_STREAM_GOLDEN)
def test_fp2_stream_reference_checksums(oracle, log2, expected):
    a, b = spike.fp2_inputs(1 << log2)
    assert oracle.fnv(oracle.fp2_mul_stream(a, b)) == expected


@pytest.mark.parametrize("log2,rounds,expected", spike.FP2_CHAIN_GOLDEN)
def test_fp2_chain_reference_checksums(oracle, log2, rounds, expected):
    a, b = spike.fp2_inputs(1 << log2)
    assert oracle.fnv(oracle.fp2_chain(a, b, rounds)) == expected


# ---- FpStream / ChaCha8 ---------------------------------------------------------------

KAT_SEED = bytes((17 * i + 3) % 256 for i in range(32))


def test_chacha8_reference_kat(oracle):
    # rust/volta-accel/src/lib.rs:7517-7528: 6th raw u64 is 0xffffffffb1461b28
    raw = oracle.raw_u64(KAT_SEED, 0x19664BCA, 8)
    assert int(raw[5]) == 0xFFFF_FFFF_B146_1B28
    rows = oracle.fp_rows(KAT_SEED, 0x19664BCA, 3, 10)
    # that draw is >= p and must be rejected, so row 0 takes raw[6] at index 5
    assert rows[0, :5].tolist() == raw[:5].tolist()
    assert int(rows[0, 5]) == int(raw[6])
    assert (rows < P).all()


def test_chacha8_published_zero_key_keystream(oracle):
    # Bernstein ChaCha, 8 rounds, 256-bit all-zero key, zero nonce: the
    # published keystream's blocks 0 and 1 (block counter 0 and 1), so the
    # counter increment and the second block's word order are pinned too.
    raw = oracle.raw_u64(bytes(32), 0, 16)
    ks = raw.view(np.uint8).tobytes().hex()
    assert ks[:128] == (
        "3e00ef2f895f40d67f5bb8e81f09a5a12c840ec3ce9a7f3b181be188ef711a1e"
        "984ce172b9216f419f445367456d5619314a42a3da86b001387bfdb80e0cfe42")
    assert ks[128:] == (
        "d2aefa0deaa5c151bf0adb6c01f2a5adc0fd581259f9a2aadcf20f8fd566a26b"
        "5032ec38bbc5da98ee0c6f568b872a65a08abf251deb21bb4b56e5d8821e68aa")


def test_stream_domain_separation_and_fp2(oracle):
    seed = bytes([42] * 32)
    a = oracle.fp_rows(seed, 7, 1, 32)[0]
    b = oracle.fp_rows(seed, 7, 1, 32)[0]
    c = oracle.fp_rows(seed, 8, 1, 32)[0]
    assert (a == b).all() and not (a == c).all()
    # next_fp2 = two consecutive accepted draws (c0 then c1)
    f2 = oracle.fp2_rows_padded(seed, 7, 1, 4, 6)[0]
    assert f2[:4].reshape(-1).tolist() == a[:8].tolist()
    assert f2[4:].reshape(-1).tolist() == [0, 0, 0, 0]
    # the second block continues the keystream (counter increments)
    raw = oracle.raw_u64(seed, 7, 16)
    assert raw[:8].tolist() != raw[8:].tolist()


def test_gather_columns(oracle):
    m = np.arange(24, dtype=np.uint64).reshape(4, 6)
    idx = np.array([5, 0, 3], dtype=np.uint32)
    assert oracle.gather_columns(m, idx).tolist() == [m[:, 5].tolist(), m[:, 0].tolist(), m[:, 3].tolist()]


# ---- BLAKE3 column leaves and Merkle tree -------------------------------------------

def test_blake3_published_digests(oracle):
    for msg, want in spike.BLAKE3_PUBLISHED:
        assert oracle.blake3(msg).hex() == want


def test_merkle16_reference_root(oracle):
    """rust/volta-pcs/src/merkle.rs:89-96: 1-byte leaves and 64-byte pair hashes."""
    leaves = np.frombuffer(b"".join(oracle.blake3(bytes([i])) for i in range(16)), np.uint8).reshape(16, 32)
    assert oracle.merkle_tree(leaves)[-1].tobytes() == spike.MERKLE16_ROOT


@pytest.mark.parametrize("rows,cols,want", spike.MERKLE_BENCH_GOLDEN)
def test_merkle_bench_reference_roots(oracle, rows, cols, want):
    """One 256-byte chunk per column (32 rows) and 8 chunks per column (1024 rows)."""
    m = oracle.merkle_bench_matrix(rows, cols)
    assert (m.reshape(rows, cols) == spike.merkle_bench_matrix(rows, cols)).all()
    leaves = oracle.hash_fp_columns(m, rows, cols)
    assert oracle.merkle_tree(leaves)[-1].tobytes().hex() == want


def test_column_leaf_bytes_are_le_words_row_by_row(oracle):
    """A leaf hashes column j's values as LE u64 row by row, an Fp2 as c0 then c1
    (ligero.rs:351-357): a transposed or word-swapped gather fails."""
    rnd = np.random.default_rng(5)
    m = rnd.integers(0, P, size=(9, 4), dtype=np.uint64)
    leaves = oracle.hash_fp_columns(m, 9, 4)
    for j in range(4):
        assert leaves[j].tobytes() == oracle.blake3(b"".join(int(x).to_bytes(8, "little") for x in m[:, j]))
    m2 = rnd.integers(0, P, size=(5, 2, 2), dtype=np.uint64)
    leaves2 = oracle.hash_fp2_columns(m2, 5, 2)
    for j in range(2):
        data = b"".join(int(m2[i, j, 0]).to_bytes(8, "little") + int(m2[i, j, 1]).to_bytes(8, "little")
                        for i in range(5))
        assert leaves2[j].tobytes() == oracle.blake3(data)


def _verify_path(oracle, root, idx, leaf, path):
    """merkle.rs:55-80 restated: fold the siblings from the leaf up."""
    acc = leaf
    for sib in path:
        acc = oracle.blake3(acc + sib) if idx & 1 == 0 else oracle.blake3(sib + acc)
        idx >>= 1
    return acc == root


def test_merkle_paths_verify_and_detect_tampering(oracle):
    rnd = np.random.default_rng(9)
    for n in (2, 8, 64):
        leaves = rnd.integers(0, 256, size=(n, 32), dtype=np.uint8)
        tree = oracle.merkle_tree(leaves)
        root = tree[-1].tobytes()
        idx = np.arange(n, dtype=np.uint32)
        paths = oracle.merkle_paths(tree, n, idx)
        for i in range(n):
            path = [paths[i, l].tobytes() for l in range(paths.shape[1])]
            assert _verify_path(oracle, root, i, leaves[i].tobytes(), path)
            assert not _verify_path(oracle, root, i ^ 1, leaves[i].tobytes(), path)
        bad = oracle.merkle_paths(tree, n, np.array([n, n + 5], np.uint32))
        assert not bad.any()  # out-of-range queries read as zero hashes


# ---- opening-path helpers -------------------------------------------------------------

def _f2mul(a, b):
    """(a0 + a1 phi)(b0 + b1 phi) with phi^2 = 7 (rust/volta-field/src/lib.rs:173-177)."""
    return ((a[0] * b[0] + 7 * a[1] * b[1]) % P, (a[0] * b[1] + a[1] * b[0]) % P)


def test_eq_rows_boolean_points_are_indicators(oracle):
    """A 0/1 point selects exactly the index whose bit k is coordinate k: pins
    the LSB-first bit order of the reference's expansion (.cu:2860-2871)."""
    dims = 4
    pts = np.array([[(x >> k) & 1, 0] for x in (0, 5, 10, 15) for k in range(dims)], np.uint64)
    eq = oracle.eq_rows(pts, 4, dims)
    for r, x in enumerate((0, 5, 10, 15)):
        want = np.zeros((1 << dims, 2), np.uint64)
        want[x, 0] = 1
        assert (eq[r] == want).all()


def test_eq_rows_against_big_ints_and_sum_to_one(oracle):
    rnd = random.Random(11)
    rows, dims = 3, 5
    pts = [(rnd.randrange(P), rnd.randrange(P)) for _ in range(rows * dims)]
    eq = oracle.eq_rows(np.array(pts, np.uint64), rows, dims)
    for r in range(rows):
        total = (0, 0)
        for x in range(1 << dims):
            acc = (1, 0)
            for k in range(dims):
                p = pts[r * dims + k]
                acc = _f2mul(acc, p if (x >> k) & 1 else ((1 - p[0]) % P, (-p[1]) % P))
            assert tuple(int(v) for v in eq[r, x]) == acc
            total = ((total[0] + acc[0]) % P, (total[1] + acc[1]) % P)
        assert total == (1, 0)  # sum_x eq(p, x) = prod_k (p_k + 1 - p_k) = 1
    assert (oracle.eq_rows(np.zeros((0, 2), np.uint64), 2, 0) == np.array([[[1, 0]], [[1, 0]]])).all()


def test_fp2_row_dots_against_big_ints(oracle):
    rnd = np.random.default_rng(12)
    rows, length, sa, sb = 4, 37, 40, 37
    a = rnd.integers(0, P, size=(rows * sa, 2), dtype=np.uint64)
    b = rnd.integers(0, P, size=(rows * sb, 2), dtype=np.uint64)
    got = oracle.fp2_row_dots(a, sa, b, sb, rows, length)
    for r in range(rows):
        acc = (0, 0)
        for j in range(length):
            t = _f2mul(tuple(int(v) for v in a[r * sa + j]), tuple(int(v) for v in b[r * sb + j]))
            acc = ((acc[0] + t[0]) % P, (acc[1] + t[1]) % P)
        assert tuple(int(v) for v in got[r]) == acc
