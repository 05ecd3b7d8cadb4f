"""The oracle's composed CPU commit (commit_impl, rust/volta-pcs/src/ligero.rs:543-624)
and its combine_rows restatement (ligero.rs:680-720), pinned against
independent reconstructions built here from pinned primitives: big-integer
DFTs, blake3 of hand-built column bytes (blake3 itself is pinned by the
published digests in test_oracle.py) and the Merkle pair rule of
merkle.rs:13-37."""
import random

import numpy as np
import pytest

P = 0xFFFF_FFFF_0000_0001


def naive_encode(msg, n):
    """out[j] = sum_i m_i w^(ij), w = 7^((p-1)/n) (rust/volta-pcs/src/ntt.rs:8-70)."""
    w = pow(7, (P - 1) // n, P)
    return [sum(int(m) * pow(w, i * j, P) for i, m in enumerate(msg)) % P for j in range(n)]


@pytest.mark.parametrize("rows,cols,pad,code_len", [(8, 8, 2, 16), (4, 4, 0, 8), (2, 3, 5, 16)])
def test_commit_root_matches_hand_composition(oracle, rows, cols, pad, code_len):
    rnd = random.Random(rows * 100 + cols)
    w = np.array([rnd.randrange(-32768, 32768) for _ in range(rows * cols)], dtype=np.int16)
    seed = bytes([0x79] * 32)
    root, enc, pads = oracle.commit_root(w, rows, cols, pad, code_len, seed, keep=True)
    # pads: FpStream::domain_separated(seed, r), r = 0.. (ligero.rs:555-563)
    want_pads = oracle.fp_rows(seed, 0, rows, pad) if pad else np.zeros((rows, 0), np.uint64)
    assert (pads == want_pads).all()
    # rows: NttPlan::forward of lift(w) || pads || 0 (ligero.rs:584-592)
    for r in range(rows):
        msg = [int(x) % P for x in w[r * cols:(r + 1) * cols]] + [int(x) for x in want_pads[r]]
        assert [int(x) for x in enc[r]] == naive_encode(msg, code_len)
    # leaves: blake3 of each column's LE u64 words, row by row (ligero.rs:596-616)
    leaves = [oracle.blake3(b"".join(int(enc[r, j]).to_bytes(8, "little") for r in range(rows)))
              for j in range(code_len)]
    # tree: parents blake3(left || right) up to one root (merkle.rs:13-37)
    level = leaves
    while len(level) > 1:
        level = [oracle.blake3(level[2 * i] + level[2 * i + 1]) for i in range(len(level) // 2)]
    assert root == level[0]
    assert oracle.commit_root(w, rows, cols, pad, code_len, seed) == root


def test_commit_root_depends_on_every_input(oracle):
    rows, cols, pad, code_len = 4, 4, 2, 8
    w = np.arange(rows * cols, dtype=np.int16) - 7
    seed = bytes(range(32))
    base = oracle.commit_root(w, rows, cols, pad, code_len, seed)
    w2 = w.copy()
    w2[-1] += 1
    assert oracle.commit_root(w2, rows, cols, pad, code_len, seed) != base
    assert oracle.commit_root(w, rows, cols, pad, code_len, bytes(32)) != base
    with pytest.raises(ValueError):
        oracle.commit_root(w, rows, cols, 5, code_len, seed)  # cols + pad > code_len


@pytest.mark.parametrize("rows,cols,pad,comb,threads", [(7, 203, 3, 2, 3), (3, 64, 0, 1, 16), (5, 9, 4, 3, 1),
                                                         (9, 1, 2, 2, 2)])
def test_combine_rows_chunked_walk_against_big_ints(oracle, rows, cols, pad, comb, threads):
    """combine_rows splits the data block into threads*4 column chunks (here
    also ragged, empty and single-column ones); every split gives the
    double-loop sums."""
    rnd = random.Random(rows * cols + comb)
    w = np.array([rnd.randrange(-32768, 32768) for _ in range(rows * cols)], dtype=np.int16)
    pads = np.array([rnd.randrange(P) for _ in range(rows * pad)], dtype=np.uint64)
    co = np.array([[rnd.randrange(P), rnd.randrange(P)] for _ in range(comb * rows)], dtype=np.uint64)
    got = oracle.pcs_combine_rows(w, pads if pad else None, co, rows, cols, pad, comb, threads=threads)
    for k in range(comb):
        for j in range(cols + pad):
            s0 = s1 = 0
            for i in range(rows):
                x = int(w[i * cols + j]) % P if j < cols else int(pads[i * pad + j - cols])
                s0 += int(co[k * rows + i, 0]) * x
                s1 += int(co[k * rows + i, 1]) * x
            assert (int(got[k, j, 0]), int(got[k, j, 1])) == (s0 % P, s1 % P)
